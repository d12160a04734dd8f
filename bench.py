"""MoE-layer tokens/s and % of peak HBM bandwidth, Mixtral-shaped Q4_K layer at decode batch 1.

One step = one Transformer::moe_ffn pass (route, dispatch, gate/up + SwiGLU,
down, combine) over one token, through kmoe_moe_ffn. Workload: hidden 4096,
expert FFN 14336, 8 experts, top-2, Q4_K random-init experts (random
well-formed blocks, as kestrel's own synthetic models are built:
tools/make_synthetic.py:39-58), router fp32 N(0, 0.02), activations N(0, 1).

Steps rotate over NL distinct layers (NL x 793 MB of experts, default 4 =
3.2 GB) so the 256 MB Infinity Cache cannot serve repeats; every step reads
its two experts from HBM. Inputs are resident in HBM before timing starts.

Prints one JSON line (contract in the build brief): value = tokens/s of the
whole job (one GPU), roofline of the dominant kernel (its duration measured
live with HIP events attached to its own dispatch, hipExtLaunchKernelGGL on
the library's stream; its HBM traffic from the committed rocprofv3 counter
passes), cpu_baseline = the oracle (C++ restatement of kestrel's AVX2 path)
timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from tests.helpers import (DSV2LITE, MOE6B, stack_bytes_per_token, stack_model,  # noqa: E402
                           synthetic_blocks, tensor_bytes)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
D, FF, E, K = 4096, 14336, 8, 2
Q8_0, Q4_K, Q6_K = 8, 12, 14
ROW_GU = 4096 // 256 * 144   # 2304 B per gate/up row
ROW_DN = 14336 // 256 * 144  # 8064 B per down row
PART = FF * ROW_GU           # 33,030,144 B (gate, up and down parts are equal)
EXPERT_BYTES = 3 * PART      # 99,090,432 B


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--layers", type=int, default=4, help="distinct layers rotated through (793 MB each)")
    ap.add_argument("--tokens", type=int, default=1, help="tokens per step (decode batch)")
    ap.add_argument("--regime", type=int, default=0)
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of a replayed HIP graph")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--pcie-steps", type=int, default=200,
                    help="steps of the host-buffer variant (h copied in, out copied back, synchronous)")
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="tokens of the prefill leg (int8 matrix-core path); 0 skips it")
    ap.add_argument("--prefill-steps", type=int, default=40)
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the other measured rows (decode b=8/32, dense Q4_K/Q6_K matvec, Q4_K_M-mix "
                         "decode, Qwen3- and DeepSeek-V2-Lite-shaped layers, expert-tier preload, decode stacks)")
    ap.add_argument("--legs", default="batches,matvec_q4k,matvec_q6k,q4k_m,qwen3,c5_layer,preload,decode_stack,"
                                      "c5_stack,measure",
                    help="comma list of the other measured rows to run (batches, matvec_q4k, matvec_q6k, "
                         "q4k_m, qwen3, c5_layer, preload, decode_stack, c5_stack, measure)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain copy kernel (torch.neg, MIB in and MIB out) 5 times and exit: "
                         "the reference point that scales FETCH_SIZE / WRITE_SIZE counters to bytes")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "moe_decode_b1_mixtral_q4k_traffic.txt")


def measured_traffic() -> dict:
    """HBM bytes per launch by library timer name, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by a plain copy kernel)."""
    out = {}
    if os.path.exists(TRAFFIC_FILE):
        for line in open(TRAFFIC_FILE):
            f = line.split()
            if f and not f[0].startswith("#") and len(f) >= 2:
                out[f[0]] = int(f[1])
    return out


def copy_probe(torch, mib: int):
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "launches": 5}))


def make_layers(ctx, torch, n_layers: int, seed: int = 0):
    """Random well-formed Q4_K experts generated on the device (f16 d and dmin
    overwritten so weights have std ~0.02 and zero mean), router N(0, 0.02)."""
    import numpy as np

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dh = np.array([1.4e-4], np.float16).view(np.uint8)
    mh = np.array([7.5 * 1.4e-4], np.float16).view(np.uint8)
    hdr = torch.tensor(np.concatenate([dh, mh]), dtype=torch.uint8, device="cuda")
    rng = np.random.default_rng(seed)
    for l in range(n_layers):
        ctx.layer_create(l, E, K, D, FF, Q4_K, Q4_K, Q4_K, True, 0.0)
        ctx.router_upload(l, (rng.standard_normal((E, D)) * 0.02).astype(np.float32))
        for e in range(E):
            for p in range(3):
                t = torch.randint(0, 256, (PART // 144, 144), dtype=torch.uint8, device="cuda", generator=g)
                t[:, 0:4] = hdr
                ctx.expert_upload(l, e, p, t)
                del t
    torch.cuda.synchronize()


def host_cpu() -> dict:
    """This host's CPU model and the hardware threads and physical cores this
    process may run on (its affinity mask; kestrel's default thread count is
    the physical core count, README.md:487)."""
    aff = set(os.sched_getaffinity(0))
    model, cores, cur = None, set(), {}
    try:
        lines = open("/proc/cpuinfo").read().splitlines() + [""]
    except OSError:
        lines = []
    for line in lines:
        if not line.strip():
            if cur and int(cur.get("processor", -1)) in aff:
                cores.add((cur.get("physical id", "0"), cur.get("core id", cur.get("processor"))))
                model = model or cur.get("model name")
            cur = {}
            continue
        k, _, v = line.partition(":")
        cur[k.strip()] = v.strip()
    return {"cpu_model": model, "hw_threads": len(aff), "physical_cores": len(cores) or len(aff)}


def cpu_threads(cap: int) -> int:
    """kestrel's default: one thread per physical core (capped)."""
    return max(1, min(cap, host_cpu()["physical_cores"]))


def timed_calls(fn, seconds: float, max_calls: int):
    """Calls fn(i) until `seconds` or `max_calls`; returns (calls, elapsed s)."""
    fn(0)  # warm
    t0 = time.perf_counter()
    n = 0
    while True:
        fn(n)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= max_calls:
            return n, el


def cpu_baseline(ctx, torch, seconds: float, threads: int):
    """Oracle moe_ffn (C++ restatement of kestrel's AVX2 path, transformer.rs:513)
    on layer 0's exact bytes, one token per call, for about `seconds` with one
    thread per physical core, then about a third of that on one thread."""
    import numpy as np

    from oracle import pyoracle as orc

    parts = [[ctx.expert_read(0, e, p) for p in range(3)] for e in range(E)]
    rng = np.random.default_rng(0)
    router = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)  # same stream as make_layers' layer 0
    L = orc.Layer(E, K, D, FF, Q4_K, Q4_K, Q4_K, router, [p[0] for p in parts], [p[1] for p in parts],
                  [p[2] for p in parts], True, 0.0)
    info = host_cpu()
    nthreads = cpu_threads(threads)
    h = rng.standard_normal((64, D)).astype(np.float32)
    n, el = timed_calls(lambda i: L.moe_ffn(h[i % 64:i % 64 + 1], threads=nthreads), seconds, 5000)
    n1, el1 = timed_calls(lambda i: L.moe_ffn(h[i % 64:i % 64 + 1], threads=1), seconds / 3, 1000)
    gemv = orc.bench_gemv(Q4_K, 2048, 4096, 50, nthreads)  # quant.rs:348-368 metric
    gemv1 = orc.bench_gemv(Q4_K, 2048, 4096, 20, 1)
    return {
        "value": round(n / el, 3),
        "unit": "tokens/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"{n} single-token moe_ffn calls on layer 0 (Mixtral shape, Q4_K, AVX2 regime), {el:.1f} s, "
                  f"{nthreads} threads (one per physical core)",
        **info,
        "one_thread": {"value": round(n1 / el1, 3), "unit": "tokens/s", "sample": f"{n1} calls, {el1:.1f} s"},
        "gemv_q4k_2048x4096_GBps": round(gemv / 1e9, 3),
        "gemv_q4k_2048x4096_GBps_one_thread": round(gemv1 / 1e9, 3),
    }


# Kernel names the library's timing mode reports (kmoe_profile_read).
PROFILE_NAMES = ("add_rows", "argmax", "attention", "attention_q8", "block_sums_q4k", "block_sums_q4k_mfma",
                 "block_sums_q6k", "block_sums_q8_0", "combine", "dequant_x", "dispatch", "f32_rows_plain", "gemm_f32", "get_rows",
                 "kv_store", "matmul_f32_ordered", "matvec_q4k", "matvec_q4k_mfma", "matvec_q6k", "matvec_q8_0",
                 "matvec_qkv_rope", "matvec_unpacked", "moe_down_dec", "moe_down_f32", "moe_down_f32_rows", "moe_down_few",
                 "moe_down_int", "moe_down_shared", "moe_gate_up_few",
                 "moe_down_mfma", "moe_down_small", "moe_gate_f32", "moe_gate_up_dec", "moe_gate_up_f32_rows", "moe_gate_up_int",
                 "moe_gate_up_mfma", "moe_gate_up_small", "moe_up_f32", "pos_advance", "quant_q8", "quant_q8k",
                 "quant_slots_q8", "quant_slots_q8k", "quant_slots_shared", "rmsnorm", "rmsnorm_quant", "rope", "rope_kv",
                 "route_decode", "route_topk", "router_logits", "shared_add", "shared_down_add", "shared_gate", "shared_gate_up_f32",
                 "shared_swiglu", "shared_swiglu_quant", "swiglu")

INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix-core peak, TOP/s


def prefill_leg(ctx, torch, a):
    """Prefill: S tokens per moe_ffn step on the int path for every row (the
    int8 matrix-core kernels), rotating over the same layers, replayed as a HIP
    graph. Reports tokens/s, the matrix-core utilisation of the grouped
    kernels (algorithmic int8 ops: 2 per multiply-add of the top-k expert
    products, over their measured durations) and HBM bytes touched."""
    S = a.prefill_tokens
    ctx.set_regime(1)
    ctx.set_stream(torch.cuda.current_stream())
    hp = torch.randn((a.layers, S, D), dtype=torch.float32, device="cuda")
    op = torch.empty((a.layers, S, D), dtype=torch.float32, device="cuda")

    def step(i):
        l = i % a.layers
        ctx.moe_ffn(l, hp[l], op[l])

    for i in range(a.layers * 2):
        step(i)
    torch.cuda.synchronize()
    ctx.profile_enable(True)
    for i in range(a.layers * 4):
        step(i)
    torch.cuda.synchronize()
    kern = {}
    for n in ["router_logits", "route_topk", "dispatch", "quant_q8k", "moe_gate_up_mfma", "moe_gate_up_int",
              "quant_slots_q8k", "moe_down_mfma", "moe_down_int", "combine"]:
        ms, cnt = ctx.profile_read(n)
        if cnt:
            kern[n] = {"avg_us": round(ms * 1000.0 / cnt, 3), "launches": cnt}
    ctx.profile_enable(False)
    whole = None
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            ctx.set_stream(s)
            for l in range(a.layers):
                step(l)
        torch.cuda.current_stream().wait_stream(s)
        whole = torch.cuda.CUDAGraph()
        with torch.cuda.graph(whole):
            ctx.set_stream(torch.cuda.current_stream())
            for l in range(a.layers):
                step(l)
        ctx.set_stream(torch.cuda.current_stream())
        for l in range(a.layers):
            step(l)
        torch.cuda.synchronize()
        ref = op.clone()
        for _ in range(2):
            op.zero_()
            whole.replay()
            torch.cuda.synchronize()
            if not torch.equal(ref, op):
                raise RuntimeError("prefill graph replay differs from eager")
    except Exception as ex:
        print(f"# prefill graph capture unavailable: {ex}", file=sys.stderr)
        whole = None
        ctx.set_stream(torch.cuda.current_stream())
    n_rep = max(1, a.prefill_steps // a.layers)

    def run(nr):
        for _ in range(nr):
            if whole is not None:
                whole.replay()
            else:
                for l in range(a.layers):
                    step(l)

    run(2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(n_rep)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    steps = n_rep * a.layers
    ms_step = el * 1000.0 / steps
    ops_gu = 2.0 * S * K * 2 * D * FF  # gate and up products of the routed rows
    ops_dn = 2.0 * S * K * D * FF
    util = {}
    for name, ops in (("moe_gate_up_mfma", ops_gu), ("moe_down_mfma", ops_dn)):
        if name in kern:
            tops = ops / (kern[name]["avg_us"] * 1e-6) / 1e12
            util[name] = {"alg_ops": ops, "avg_us": kern[name]["avg_us"], "achieved_TOPs": round(tops, 1),
                          "frac": round(tops / INT8_PEAK_TOPS, 4)}
    mf_us = sum(kern[n]["avg_us"] for n in ("moe_gate_up_mfma", "moe_down_mfma") if n in kern)
    touched = E * EXPERT_BYTES + E * D * 4
    # The reference's own prefill arithmetic (AVX2 regime: experts with >= 4
    # rows dequantize to f32 and run the f32 GEMM, quant.rs:242-260), on the
    # same inputs: its GPU time, and how far the int8 path's outputs are from it.
    o_int = op.clone()
    ctx.set_regime(0)
    t_avx = graph_time(torch, ctx, [lambda l=l: step(l) for l in range(a.layers)], max(1, n_rep // 2)) / a.layers
    for l in range(a.layers):
        step(l)
    torch.cuda.synchronize()
    o_f32 = op.clone()
    ctx.set_regime(1)
    rel = max(float(((o_int[l] - o_f32[l]).double().norm() / o_f32[l].double().norm()).item())
              for l in range(a.layers))
    res = {
        "tokens": S,
        "steps": steps,
        "tokens_per_s": round(S * steps / el, 1),
        "ms_per_step": round(ms_step, 5),
        "regime": "int8",
        "launch": "hip-graph" if whole is not None else "eager",
        "mfma": {"bound": "mfma", "unit": "TOP/s", "peak": INT8_PEAK_TOPS,
                 "achieved": round((ops_gu + ops_dn) / (mf_us * 1e-6) / 1e12, 1) if mf_us else None,
                 "frac": round((ops_gu + ops_dn) / (mf_us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4) if mf_us else None,
                 "alg_ops_per_step": ops_gu + ops_dn, "kernels": util},
        "layer_TOPs": round((ops_gu + ops_dn) / (ms_step * 1e-3) / 1e12, 1),
        "hbm_touched_GBps": round(touched / (ms_step * 1e-3) / 1e9, 1),
        "hbm_frac": round(touched / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "kernels_us": kern,
        "avx2_regime": {"tokens_per_s": round(S / t_avx, 1), "ms_per_step": round(t_avx * 1e3, 5),
                        "launch": "hip-graph", "arithmetic": "f32 GEMM on dequantized weights for experts with "
                                                             ">= 4 rows (every expert at this batch)"},
        "int8_vs_f32_rel_l2": round(rel, 6),
        "cpu_baseline": None,
    }
    ctx.set_regime(a.regime)
    return res


def graph_time(torch, ctx, fns, reps: int) -> float:
    """Seconds per run of fns (library launches on the current stream), captured
    once as a HIP graph after an eager run that sizes the workspace."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ctx.set_stream(s)
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.set_stream(torch.cuda.current_stream())
        for f in fns:
            f()
    ctx.set_stream(torch.cuda.current_stream())
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    el = (time.perf_counter() - t0) / reps
    del g
    return el


def batch_leg(ctx, torch, layers: int, S: int, regime: int):
    """Mixtral-shaped decode at S tokens per step over the rotated layers; HBM
    bytes from the distinct experts each layer's routing touched."""
    ctx.set_regime(regime)
    ctx.set_stream(torch.cuda.current_stream())
    hp = torch.randn((layers, S, D), dtype=torch.float32, device="cuda")
    op = torch.empty_like(hp)
    touched = []
    for l in range(layers):
        ctx.moe_ffn(l, hp[l], op[l])
        idx = ctx.last_routing(S, K, E)[0]
        touched.append(len(set(idx.cpu().numpy().ravel().tolist())))
    t = graph_time(torch, ctx, [lambda l=l: ctx.moe_ffn(l, hp[l], op[l]) for l in range(layers)], 20) / layers
    tb = (sum(touched) / layers) * EXPERT_BYTES + E * D * 4
    ctx.set_regime(0)
    return {"tokens": S, "regime": ["avx2", "int8", "exact"][regime], "tokens_per_s": round(S / t, 1),
            "ms_per_step": round(t * 1e3, 5), "experts_touched": sum(touched) / layers,
            "hbm_touched_GBps": round(tb / t / 1e9, 1), "hbm_frac": round(tb / t / 1e9 / HBM_PEAK_GBPS, 4)}


def matvec_leg(ctx, torch, wtype: int = Q4_K, pool_bytes: float = 2.2e9, cpu_seconds: float = 0.0,
               cpu_cap: int = 16):
    """Dense Q4_K or Q6_K matvec at decode batch 1 (quant::matmul, one
    activation row) over a pool of distinct weight copies larger than the
    Infinity Cache: the whole call (Q8_K of x, then the matvec) replayed as a
    graph, the matvec kernel's own time, and (cpu_seconds > 0) the oracle's
    GEMV at the same shape on this host."""
    import numpy as np

    from kestrel_amd import kmoe

    ctx.set_regime(0)
    if wtype == Q4_K:  # f16 d, dmin at bytes 0-3: weights of std ~0.02
        blk, off = 144, 0
        hdr = np.concatenate([np.array([1.4e-4], np.float16).view(np.uint8),
                              np.array([7.5 * 1.4e-4], np.float16).view(np.uint8)])
    else:  # Q6_K: f16 d at bytes 208-209
        blk, off = 210, 208
        hdr = np.array([1.5e-5], np.float16).view(np.uint8)
    hdr = torch.tensor(hdr, dtype=torch.uint8, device="cuda")
    out = {}
    for rows, cols in ((4096, 4096), (14336, 4096), (4096, 14336)):
        nbytes = rows * (cols // 256) * blk
        copies = int(-(-pool_bytes // nbytes))
        pool = torch.randint(0, 256, (copies, nbytes // blk, blk), dtype=torch.uint8, device="cuda")
        pool[:, :, off:off + hdr.numel()] = hdr
        x = torch.randn((1, cols), dtype=torch.float32, device="cuda")
        y = torch.empty((1, rows), dtype=torch.float32, device="cuda")
        lib = ctx.lib

        def call(i):
            ctx.check(lib.kmoe_matmul(ctx.h, wtype, kmoe._ptr(pool[i]), nbytes, rows, cols, kmoe._ptr(x), 1,
                                      kmoe._ptr(y)))

        t = graph_time(torch, ctx, [lambda i=i: call(i) for i in range(copies)], 5) / copies
        b = nbytes + cols * 4 + rows * 4
        # the matvec kernel alone (its own dispatch timestamps), beside the
        # activation quantization that precedes it in the call
        ctx.profile_enable(True)
        for i in range(copies):
            call(i)
        torch.cuda.synchronize()
        kname = "matvec_q4k" if wtype == Q4_K else "matvec_q6k"
        ms_k, n_k = ctx.profile_read(kname)
        ms_q, n_q = ctx.profile_read("quant_q8k")
        ctx.profile_enable(False)
        k_us = ms_k * 1e3 / max(1, n_k)
        # algorithmic bytes of the kernel: the weights, the Q8_K row (cols + cols/16*4 + cols/256*4) and out;
        # when no quantization kernel ran, the kernel read the f32 row (cols*4) and quantized it itself
        xb = cols * 4 if n_q == 0 else cols + cols // 16 * 4 + cols // 256 * 4
        kb = nbytes + xb + rows * 4
        row = {"us": round(t * 1e6, 3), "GBps": round(b / t / 1e9, 1), "frac": round(b / t / 1e9 / HBM_PEAK_GBPS, 4),
               "pool_copies": copies,
               "kernel": {"name": kname, "avg_us": round(k_us, 3), "alg_bytes": kb,
                          "GBps": round(kb / (k_us * 1e-6) / 1e9, 1),
                          "frac": round(kb / (k_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                          "quant_q8k_us": round(ms_q * 1e3 / max(1, n_q), 3)}}
        if cpu_seconds > 0:  # the reference's GEMV metric at this shape (quant.rs:348-368)
            from oracle import pyoracle as orc

            nt = cpu_threads(cpu_cap)
            it = max(2, int(cpu_seconds * 20e9 / nbytes / 4))
            g = orc.bench_gemv(wtype, rows, cols, it, nt)
            g1 = orc.bench_gemv(wtype, rows, cols, max(2, it // 8), 1)
            row["cpu_baseline"] = {"value": round(g / 1e9, 3), "unit": "GB/s", "cores": nt, "kind": "port",
                                   "one_thread_GBps": round(g1 / 1e9, 3),
                                   "sample": f"quant::matmul at one row, {it} calls on one {rows}x{cols} matrix "
                                             f"(xorshift bytes & 0x3f, activations (i % 7) * 0.01)"}
        out[f"{rows}x{cols}"] = row
        del pool
    torch.cuda.empty_cache()
    return out


def q4km_leg(ctx, torch, layers: int = 4, seed: int = 2):
    """Mixtral-shaped decode at batch 1 with the tensor mix of a Q4_K_M file:
    Q4_K gate/up, Q6_K down (48,168,960 B per expert), random well-formed
    blocks, router N(0, 0.02); layers rotated past the Infinity Cache."""
    import numpy as np

    h4 = torch.tensor(np.concatenate([np.array([1.4e-4], np.float16).view(np.uint8),
                                      np.array([7.5 * 1.4e-4], np.float16).view(np.uint8)]),
                      dtype=torch.uint8, device="cuda")
    h6 = torch.tensor(np.array([1.5e-5], np.float16).view(np.uint8), dtype=torch.uint8, device="cuda")
    down6 = D * (FF // 256) * 210
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    base = 200
    for l in range(layers):
        ctx.layer_create(base + l, E, K, D, FF, Q4_K, Q4_K, Q6_K, True, 0.0)
        ctx.router_upload(base + l, (rng.standard_normal((E, D)) * 0.02).astype(np.float32))
        for e in range(E):
            for p in range(2):
                t = torch.randint(0, 256, (PART // 144, 144), dtype=torch.uint8, device="cuda", generator=g)
                t[:, 0:4] = h4
                ctx.expert_upload(base + l, e, p, t)
            t = torch.randint(0, 256, (down6 // 210, 210), dtype=torch.uint8, device="cuda", generator=g)
            t[:, 208:210] = h6
            ctx.expert_upload(base + l, e, 2, t)
            del t
    torch.cuda.synchronize()
    ctx.set_stream(torch.cuda.current_stream())
    hp = torch.randn((layers, 1, D), dtype=torch.float32, device="cuda")
    op = torch.empty_like(hp)
    for l in range(layers):
        ctx.moe_ffn(base + l, hp[l], op[l])
    t = graph_time(torch, ctx, [lambda l=l: ctx.moe_ffn(base + l, hp[l], op[l]) for l in range(layers)], 100)
    t /= layers
    tb = K * (2 * PART + down6) + E * D * 4
    for l in range(layers):
        ctx.layer_destroy(base + l)
    torch.cuda.empty_cache()
    return {"tokens": 1, "weights": "Q4_K gate/up, Q6_K down", "tokens_per_s": round(1 / t, 1),
            "us_per_step": round(t * 1e6, 2), "bytes_per_token": tb, "hbm_GBps": round(tb / t / 1e9, 1),
            "hbm_frac": round(tb / t / 1e9 / HBM_PEAK_GBPS, 4)}


def preload_leg(ctx, torch, reps: int = 3):
    """Filling the HBM expert tier (ExpertStore::preload_all): one
    Mixtral-shaped Q4_K_M layer (Q4_K gate/up, Q6_K down, 8 experts, 915 MB
    of extents) preloaded from a model image in host memory, laid out as a
    prepared KGUF (one copy per expert) and as a plain GGUF (three), from
    pageable and from pinned memory, beside one plain pinned host-to-device
    copy of the same bytes. Rates are expert bytes per second, PCIe included."""
    import numpy as np

    page, align = 4096, 32
    au = lambda v, a: (v + a - 1) // a * a
    s = [PART, PART, D * (FF // 256) * 210]
    o = [0, au(s[0], align)]
    o.append(au(o[1] + s[1], align))
    stride = au(o[2] + s[2], page)
    expert_bytes = E * sum(s)
    pinned = torch.empty(E * stride, dtype=torch.uint8, pin_memory=True)
    pinned.fill_(0x5A)
    img = np.full(E * stride, 0x5A, np.uint8)
    gguf_off = [0, E * s[0], E * (s[0] + s[1])]
    lid = 300

    def run(image, off, strides):
        ctx.layer_create(lid, E, K, D, FF, Q4_K, Q4_K, Q6_K, True, 0.0)
        try:
            ts, copies = [], 0
            for _ in range(reps):
                t0 = time.perf_counter()
                copies = ctx.layer_preload(lid, image, off, strides)
                ts.append(time.perf_counter() - t0)
        finally:
            ctx.layer_destroy(lid)
        t = sorted(ts)[len(ts) // 2]
        return {"copies": copies, "ms": round(t * 1e3, 2), "GBps": round(expert_bytes / t / 1e9, 2)}

    out = {"expert_bytes": expert_bytes, "layout_stride": stride}
    out["kgguf_pageable"] = run(img, [x for x in o], [stride] * 3)
    out["gguf_pageable"] = run(img[:expert_bytes], gguf_off, s)
    out["kgguf_pinned"] = run(pinned.numpy(), [x for x in o], [stride] * 3)
    dst = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    ts = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dst.copy_(pinned, non_blocking=True)
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    out["h2d_pinned_copy_GBps"] = round(E * stride / t / 1e9, 2)
    del dst, pinned
    torch.cuda.empty_cache()
    return out


def decode_stack_leg(ctx, torch, c: dict, prompt: int = 128, steps: int = 256, cpu_seconds: float = 0.0,
                     cpu_cap: int = 16):
    """A whole decode stack on the GPU through Decoder (Transformer::forward),
    every weight resident in HBM: a 128-token prompt of uniform random ids,
    then greedy decode steps, each one token through all layers, the head and
    argmax, replayed as one HIP graph. c: MOE6B (kestrel's synthetic `moe-6b`,
    tools/make_synthetic.py:27) or DSV2LITE. Random well-formed blocks; expert,
    attention and dense-FFN bytes are shared between layers on the host (each
    layer still gets its own copy in HBM); routers differ per layer.

    Then a per-kernel pass (eager single-token steps, each launch timed at its
    dispatch) names the kernels that take the step's time, and with
    cpu_seconds > 0 the oracle's Transformer (the C++ restatement of kestrel's
    AVX2 path) decodes the same model on this host's cores as the CPU
    baseline."""
    import numpy as np

    from kestrel_amd.decoder import Decoder

    L, V = c["layers"], c["vocab"]
    rng = np.random.default_rng(11)
    hp, T = stack_model(c, rng, n_ctx=prompt + steps + 8)
    ctx.set_stream(torch.cuda.current_stream())
    t0 = time.perf_counter()
    dec = Decoder(ctx, hp, T)
    torch.cuda.synchronize()
    load_s = time.perf_counter() - t0
    try:
        ids = rng.integers(0, V, prompt).tolist()
        dec.forward(ids[:8])  # sizes the workspaces; its positions are then reset
        dec.cached = 0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = dec.forward(ids)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        first = int(torch.argmax(logits).item())
        dec.decode_greedy(first, 4)  # captures the step graph, warms it
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks = dec.decode_greedy(first, steps - 4)
        torch.cuda.synchronize()
        dec_s = time.perf_counter() - t0
        n_distinct = int(torch.unique(toks).numel())
        # per-kernel pass: eager steps from the same position, every launch timed
        nprof = 8
        dec.cached = prompt
        dec.decode_greedy(first, 2, use_graph=False)
        dec.cached = prompt
        torch.cuda.synchronize()
        ctx.profile_enable(True)
        dec.decode_greedy(first, nprof, use_graph=False)
        torch.cuda.synchronize()
        per_tok = {}
        for name in PROFILE_NAMES:
            ms, cnt = ctx.profile_read(name)
            if cnt:
                per_tok[name] = {"us_per_token": round(ms * 1e3 / nprof, 2), "launches_per_token": cnt // nprof}
        ctx.profile_enable(False)
    finally:
        dec.close()
        torch.cuda.empty_cache()
    tb = stack_bytes_per_token(c)
    n = steps - 4
    ach = tb * n / dec_s / 1e9
    top = sorted(per_tok.items(), key=lambda kv: -kv[1]["us_per_token"])
    roof = {"bound": "hbm", "scope": "whole decode step: weight bytes per token / time per token",
            "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
            "traffic": None, "bytes_per_token": tb,
            "dominant_kernel": top[0][0] if top else None,
            "kernels_per_token": dict(top[:8]),
            "kernel_sum_us_per_token": round(sum(v["us_per_token"] for _, v in top), 1)}
    res = {"model": c["name"], "layers": L, "dense_layers": c["dense_layers"], "prompt_tokens": prompt,
           "prefill_tokens_per_s": round(prompt / prefill_s, 1), "decode_steps": n,
           "decode_tokens_per_s": round(n / dec_s, 1), "ms_per_token": round(dec_s / n * 1e3, 3),
           "weight_bytes_per_token": tb, "hbm_GBps": round(ach, 1),
           "hbm_frac": round(ach / HBM_PEAK_GBPS, 4),
           "distinct_tokens": n_distinct, "load_s": round(load_s, 1), "roofline": roof}
    if cpu_seconds > 0:
        res["cpu_baseline"] = cpu_stack(hp, T, c, cpu_seconds, cpu_cap)
    return res


def cpu_stack(hp: dict, T: dict, c: dict, seconds: float, cap: int):
    """The oracle's Transformer (transformer.rs:278-467 restated over the
    AVX2-path kernels) decoding the same stack on this host: a 4-token prompt,
    then single-token greedy steps for about `seconds`, one thread per
    physical core."""
    import numpy as np

    from oracle import pyoracle as orc

    nthreads = cpu_threads(cap)
    ref = orc.Transformer(hp, T, regime=orc.REGIME_AVX2, threads=nthreads)
    l = ref.forward([1, 2, 3, 4])
    tok = [orc.argmax(l)]
    limit = hp["n_ctx"] - ref.cached
    n, el = timed_calls(lambda i: tok.append(orc.argmax(ref.forward([tok[-1]]))), seconds, limit - 1)
    return {"value": round(n / el, 3), "unit": "tokens/s", "cores": nthreads, "kind": "port",
            "sample": f"{c['name']}, {hp['n_layer']} layers: 4-token prompt, then {n + 1} greedy single-token "
                      f"steps (the first untimed), {el:.1f} s, {nthreads} threads (one per physical core)",
            "ms_per_token": round(el / n * 1e3, 2), **host_cpu()}


def qwen3_leg(ctx, torch, layers: int = 4, seed: int = 1, cpu_seconds: float = 0.0, cpu_cap: int = 16):
    """Qwen3-30B-A3B-shaped layer: hidden 2048, FFN 768, 128 experts, top-8,
    Q4_K random-init experts, router N(0, 0.02) plus a rank-1 Zipf(1.1) bias
    over a seeded expert permutation (activations N(1, 1) carry it into the
    logits). Layers rotate (4 x 340 MB) past the Infinity Cache."""
    import numpy as np

    E4, K4, D4, F4 = 128, 8, 2048, 768
    part = F4 * (D4 // 256) * 144
    dh = np.array([1.4e-4], np.float16).view(np.uint8)
    mh = np.array([7.5 * 1.4e-4], np.float16).view(np.uint8)
    hdr = torch.tensor(np.concatenate([dh, mh]), dtype=torch.uint8, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    base = 100
    routers = []
    for l in range(layers):
        ctx.layer_create(base + l, E4, K4, D4, F4, Q4_K, Q4_K, Q4_K, True, 0.0)
        router = rng.standard_normal((E4, D4)) * 0.02
        rank = rng.permutation(E4) + 1
        router += (-1.1 * np.log(rank.astype(np.float64)) / D4)[:, None]
        routers.append(router.astype(np.float32))
        ctx.router_upload(base + l, routers[-1])
        for e in range(E4):
            for p in range(3):
                t = torch.randint(0, 256, (part // 144, 144), dtype=torch.uint8, device="cuda", generator=g)
                t[:, 0:4] = hdr
                ctx.expert_upload(base + l, e, p, t)
    torch.cuda.synchronize()
    expert_bytes = 3 * part
    res = []
    for S, regime in ((1, 0), (16, 0), (128, 0), (512, 0), (2048, 0), (512, 1), (2048, 1)):
        ctx.set_regime(regime)
        ctx.set_stream(torch.cuda.current_stream())
        hp = torch.randn((layers, S, D4), dtype=torch.float32, device="cuda") + 1.0
        op = torch.empty_like(hp)
        touched = []
        for l in range(layers):
            ctx.moe_ffn(base + l, hp[l], op[l])
            idx = ctx.last_routing(S, K4, E4)[0]
            touched.append(len(set(idx.cpu().numpy().ravel().tolist())))
        reps = 50 if S <= 128 else 10
        t = graph_time(torch, ctx, [lambda l=l: ctx.moe_ffn(base + l, hp[l], op[l]) for l in range(layers)], reps)
        t /= layers
        tb = (sum(touched) / layers) * expert_bytes + E4 * D4 * 4
        row = {"tokens": S, "regime": ["avx2", "int8", "exact"][regime], "tokens_per_s": round(S / t, 1),
               "us_per_step": round(t * 1e6, 2), "experts_touched": sum(touched) / layers,
               "hbm_touched_GBps": round(tb / t / 1e9, 1), "hbm_frac": round(tb / t / 1e9 / HBM_PEAK_GBPS, 4)}
        if S == 1:  # per-kernel times (their own dispatch timestamps) and the gate/up kernel's roofline
            ctx.profile_enable(True)
            for i in range(layers * 10):
                ctx.moe_ffn(base + i % layers, hp[i % layers], op[i % layers])
            torch.cuda.synchronize()
            kern = {}
            for n in ("route_decode", "moe_gate_up_dec", "quant_slots_q8k", "moe_down_dec"):
                ms, cnt = ctx.profile_read(n)
                if cnt:
                    kern[n] = {"avg_us": round(ms * 1000.0 / cnt, 3), "launches": cnt}
            ctx.profile_enable(False)
            row["kernels_us"] = kern
            if "moe_gate_up_dec" in kern:
                # 8 experts x (gate + up) rows, the Q8_K row of x, h out
                alg = K4 * 2 * part + (D4 + D4 // 16 * 4 + D4 // 256 * 4) + K4 * F4 * 4
                ach = alg / (kern["moe_gate_up_dec"]["avg_us"] * 1e-6) / 1e9
                row["roofline"] = {"bound": "hbm", "kernel": "moe_gate_up_dec", "achieved": round(ach, 1),
                                   "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                                   "alg_bytes_per_launch": alg}
            if cpu_seconds > 0:  # the oracle's moe_ffn on layer 0's bytes, one token per call
                from oracle import pyoracle as orc

                parts = [[ctx.expert_read(base, e, p) for p in range(3)] for e in range(E4)]
                L4 = orc.Layer(E4, K4, D4, F4, Q4_K, Q4_K, Q4_K, routers[0], [p[0] for p in parts],
                               [p[1] for p in parts], [p[2] for p in parts], True, 0.0)
                hx = (rng.standard_normal((64, D4)) + 1.0).astype(np.float32)
                nt = cpu_threads(cpu_cap)
                n, el = timed_calls(lambda i: L4.moe_ffn(hx[i % 64:i % 64 + 1], threads=nt), cpu_seconds, 20000)
                row["cpu_baseline"] = {"value": round(n / el, 2), "unit": "tokens/s", "cores": nt, "kind": "port",
                                       "sample": f"{n} single-token moe_ffn calls on layer 0 (AVX2 regime), "
                                                 f"{el:.1f} s"}
        res.append(row)
    ctx.set_regime(0)
    for l in range(layers):
        ctx.layer_destroy(base + l)
    torch.cuda.empty_cache()
    return res


def c5_layer_leg(ctx, torch, layers: int = 4, seed: int = 5, cpu_seconds: float = 0.0, cpu_cap: int = 16):
    """DeepSeek-V2-Lite-shaped MoE layer (the MoE layer of config 5): hidden
    2048, 64 routed experts of FFN 1408, top-6, softmax weights not
    renormalised; Q4_K gate/up, Q8_0 routed down (1408 columns need a
    32-element block type); 2 shared experts as one ungated ffn_*_shexp FFN of
    2816 (Q4_K gate/up, Q6_K down). Random well-formed blocks (weights std
    ~0.02), router N(0, 0.02), layers rotated (4 x 415 MB) past the Infinity
    Cache. Decode batch 1 (with per-kernel times, the gate/up kernel's
    roofline and the oracle on this host), 8 and 128 tokens."""
    import numpy as np

    E5, K5, D5, F5, FS = 64, 6, 2048, 1408, 2816
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    h4 = torch.tensor(np.concatenate([np.array([1.4e-4], np.float16).view(np.uint8),
                                      np.array([7.5 * 1.4e-4], np.float16).view(np.uint8)]),
                      dtype=torch.uint8, device="cuda")
    h8 = torch.tensor(np.array([0.02 / 74.0], np.float16).view(np.uint8), dtype=torch.uint8, device="cuda")
    gu_b, dn_b = tensor_bytes(Q4_K, F5, D5), tensor_bytes(Q8_0, D5, F5)
    base, routers, shared = 400, [], []
    for l in range(layers):
        ctx.layer_create(base + l, E5, K5, D5, F5, Q4_K, Q4_K, Q8_0, False, 1.0)
        routers.append((rng.standard_normal((E5, D5)) * 0.02).astype(np.float32))
        ctx.router_upload(base + l, routers[-1])
        for e in range(E5):
            for p in range(2):
                t = torch.randint(0, 256, (gu_b // 144, 144), dtype=torch.uint8, device="cuda", generator=g)
                t[:, 0:4] = h4
                ctx.expert_upload(base + l, e, p, t)
            t = torch.randint(0, 256, (dn_b // 34, 34), dtype=torch.uint8, device="cuda", generator=g)
            t[:, 0:2] = h8
            ctx.expert_upload(base + l, e, 2, t)
        sh = [synthetic_blocks(Q4_K, FS * D5 // 256, 0.02, rng), synthetic_blocks(Q4_K, FS * D5 // 256, 0.02, rng),
              synthetic_blocks(Q6_K, D5 * FS // 256, 0.02, rng)]
        ctx.shared_expert(base + l, FS, (Q4_K, Q4_K, Q6_K), *sh, gate_inp=None)
        shared.append(sh)
    torch.cuda.synchronize()
    routed_b = 2 * gu_b + dn_b
    shared_b = 2 * tensor_bytes(Q4_K, FS, D5) + tensor_bytes(Q6_K, D5, FS)
    res = []
    for S, regime in ((1, 0), (8, 0), (128, 0), (128, 1)):
        ctx.set_regime(regime)
        ctx.set_stream(torch.cuda.current_stream())
        hp = torch.randn((layers, S, D5), dtype=torch.float32, device="cuda")
        op = torch.empty_like(hp)
        touched = []
        for l in range(layers):
            ctx.moe_ffn(base + l, hp[l], op[l])
            touched.append(len(set(ctx.last_routing(S, K5, E5)[0].cpu().numpy().ravel().tolist())))
        t = graph_time(torch, ctx, [lambda l=l: ctx.moe_ffn(base + l, hp[l], op[l]) for l in range(layers)],
                       50 if S <= 8 else 10) / layers
        tb = (sum(touched) / layers) * routed_b + shared_b + E5 * D5 * 4
        row = {"tokens": S, "regime": ["avx2", "int8", "exact"][regime], "tokens_per_s": round(S / t, 1),
               "us_per_step": round(t * 1e6, 2), "experts_touched": sum(touched) / layers,
               "bytes_touched": int(tb), "hbm_touched_GBps": round(tb / t / 1e9, 1),
               "hbm_frac": round(tb / t / 1e9 / HBM_PEAK_GBPS, 4)}
        if S == 1:
            ctx.profile_enable(True)
            for i in range(layers * 10):
                ctx.moe_ffn(base + i % layers, hp[i % layers], op[i % layers])
            torch.cuda.synchronize()
            kern = {}
            for n in ("route_decode", "moe_gate_up_dec", "quant_slots_q8", "moe_down_dec", "quant_q8k", "matvec_q4k",
                      "shared_swiglu", "matvec_q6k", "shared_add"):
                ms, cnt = ctx.profile_read(n)
                if cnt:
                    kern[n] = {"avg_us": round(ms * 1000.0 / cnt, 3), "launches": cnt}
            ctx.profile_enable(False)
            row["kernels_us"] = kern
            if "moe_gate_up_dec" in kern:
                alg = K5 * 2 * gu_b + (D5 + D5 // 32 * 4 + D5 // 16 * 4) + K5 * F5 * 4
                ach = alg / (kern["moe_gate_up_dec"]["avg_us"] * 1e-6) / 1e9
                row["roofline"] = {"bound": "hbm", "kernel": "moe_gate_up_dec", "achieved": round(ach, 1),
                                   "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                                   "alg_bytes_per_launch": alg}
            if cpu_seconds > 0:  # the oracle's moe_ffn + shared expert on layer 0's bytes, one token per call
                from oracle import pyoracle as orc

                parts = [[ctx.expert_read(base, e, p) for p in range(3)] for e in range(E5)]
                L5 = orc.Layer(E5, K5, D5, F5, Q4_K, Q4_K, Q8_0, routers[0], [p[0] for p in parts],
                               [p[1] for p in parts], [p[2] for p in parts], False, 1.0)
                hx = rng.standard_normal((64, D5)).astype(np.float32)
                nt = cpu_threads(cpu_cap)
                sh = shared[0]

                def one(i):
                    x = hx[i % 64:i % 64 + 1]
                    orc.shared_expert_add(L5.moe_ffn(x, threads=nt), x, D5, FS, (Q4_K, Q4_K, Q6_K), sh[0], sh[1],
                                          sh[2], None, 0, nt)

                n, el = timed_calls(one, cpu_seconds, 20000)
                row["cpu_baseline"] = {"value": round(n / el, 2), "unit": "tokens/s", "cores": nt, "kind": "port",
                                       "sample": f"{n} single-token moe_ffn + shared-expert calls on layer 0 "
                                                 f"(AVX2 regime), {el:.1f} s"}
        res.append(row)
    ctx.set_regime(0)
    for l in range(layers):
        ctx.layer_destroy(base + l)
    torch.cuda.empty_cache()
    return res


def cpu_prefill(ctx, S: int, seconds: float, threads: int):
    """Oracle moe_ffn over S tokens in the reference's default regime (AVX2:
    f32 GEMM for experts with >= 4 rows), on layer 0's bytes."""
    import numpy as np

    from oracle import pyoracle as orc

    parts = [[ctx.expert_read(0, e, p) for p in range(3)] for e in range(E)]
    rng = np.random.default_rng(0)
    router = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)
    L = orc.Layer(E, K, D, FF, Q4_K, Q4_K, Q4_K, router, [p[0] for p in parts], [p[1] for p in parts],
                  [p[2] for p in parts], True, 0.0)
    nthreads = max(1, min(threads, orc.hw_threads()))
    h = rng.standard_normal((S, D)).astype(np.float32)
    t0 = time.perf_counter()
    n = 0
    while True:
        L.moe_ffn(h, threads=nthreads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(n * S / el, 2), "unit": "tokens/s", "cores": nthreads, "kind": "port",
            "sample": f"{n} moe_ffn call(s) of {S} tokens on layer 0 (AVX2 regime: f32 GEMM for experts "
                      f"with >= 4 rows), {el:.1f} s"}


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: --gpus must be 1 (no collectives are built)"}))
        sys.exit(2)
    import numpy as np
    import torch

    from kestrel_amd.kmoe import Context

    torch.cuda.set_device(0)
    if a.copy_probe:
        copy_probe(torch, a.copy_probe)
        return
    ctx = Context(0)
    ctx.set_regime(a.regime)
    make_layers(ctx, torch, a.layers)
    S = a.tokens
    hpool = torch.randn((a.layers, S, D), dtype=torch.float32, device="cuda")
    outs = torch.empty((a.layers, S, D), dtype=torch.float32, device="cuda")

    def step(i):
        l = i % a.layers
        ctx.moe_ffn(l, hpool[l], outs[l])

    # ---- per-kernel timing pass (HIP events on the library's stream)
    for i in range(a.layers * 2):
        step(i)
    torch.cuda.synchronize()
    ctx.profile_enable(True)
    nprof = max(a.layers * 10, 40)
    for i in range(nprof):
        step(i)
    torch.cuda.synchronize()
    names = ["route_decode", "router_logits", "route_topk", "dispatch", "quant_q8k", "moe_gate_up_dec", "moe_gate_up_int",
             "quant_slots_q8k", "moe_down_dec", "moe_down_int", "moe_gate_f32", "moe_up_f32", "moe_down_f32",
             "combine"]
    kern = {}
    for n in names:
        ms, cnt = ctx.profile_read(n)
        if cnt:
            kern[n] = {"avg_us": round(ms * 1000.0 / cnt, 3), "launches": cnt}
    ctx.profile_enable(False)

    # ---- graph capture or eager. One graph holds a pass over all rotated
    # layers (consecutive MoE layers, as a decode step's graph holds them);
    # one graph per layer covers a step count that is not a multiple of it.
    graphs = None
    whole = None
    if not a.no_graph:
        try:
            graphs = []
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for l in range(a.layers):
                    ctx.set_stream(s)
                    step(l)
            torch.cuda.current_stream().wait_stream(s)
            for l in range(a.layers):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    ctx.set_stream(torch.cuda.current_stream())
                    step(l)
                graphs.append(g)
            whole = torch.cuda.CUDAGraph()
            with torch.cuda.graph(whole):
                ctx.set_stream(torch.cuda.current_stream())
                for l in range(a.layers):
                    step(l)
            ctx.set_stream(torch.cuda.current_stream())
            # replay check against eager, for both graph forms
            ref = torch.empty_like(outs)
            for l in range(a.layers):
                step(l)
            torch.cuda.synchronize()
            ref.copy_(outs)
            for form in ("per-layer", "whole"):
                outs.zero_()
                if form == "whole":
                    whole.replay()
                else:
                    for l in range(a.layers):
                        graphs[l].replay()
                torch.cuda.synchronize()
                if not torch.equal(ref, outs):
                    bad = [l for l in range(a.layers) if not torch.equal(ref[l], outs[l])]
                    raise RuntimeError(f"{form} graph replay differs from eager on layers {bad}: max |diff| "
                                       f"{(ref - outs).abs().max().item():.3e}")
        except Exception as ex:  # fall back to eager launches, and say so
            print(f"# graph capture unavailable: {ex}", file=sys.stderr)
            graphs = whole = None
            ctx.set_stream(torch.cuda.current_stream())

    def run_steps(n):
        """n consecutive steps (layers 0, 1, ... rotating)."""
        if graphs is None:
            for i in range(n):
                step(i)
            return
        for _ in range(n // a.layers):
            whole.replay()
        for l in range(n % a.layers):
            graphs[l].replay()

    run_steps(a.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_steps(a.steps)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_step = el * 1000.0 / a.steps
    tok_s = S * a.steps / el

    # ---- host-buffer variant, as the reference's moe_ffn(&[f32]) -> Vec<f32> is
    # called: pinned h copied in, the layer, out copied back, synchronous per step
    pcie = None
    if a.pcie_steps > 0:
        hh = torch.randn((a.layers, S, D), dtype=torch.float32).pin_memory()
        ho = torch.empty((a.layers, S, D), dtype=torch.float32).pin_memory()
        hd = torch.empty((S, D), dtype=torch.float32, device="cuda")
        od = torch.empty((S, D), dtype=torch.float32, device="cuda")
        ctx.set_stream(torch.cuda.current_stream())

        def host_step(i):
            l = i % a.layers
            hd.copy_(hh[l], non_blocking=True)
            ctx.moe_ffn(l, hd, od)
            ho[l].copy_(od, non_blocking=True)
            torch.cuda.current_stream().synchronize()

        for i in range(min(20, a.pcie_steps)):
            host_step(i)
        t1 = time.perf_counter()
        for i in range(a.pcie_steps):
            host_step(i)
        el1 = time.perf_counter() - t1
        pcie = {"tokens_per_s": round(S * a.pcie_steps / el1, 1), "ms_per_step": round(el1 * 1000 / a.pcie_steps, 5),
                "steps": a.pcie_steps, "launch": "eager, synchronous per step, pinned host buffers"}

    # touched bytes per step: distinct experts of this batch (2 at b=1) + router
    touched = 2 * EXPERT_BYTES + E * D * 4 if S == 1 else None
    gu_name = "moe_gate_up_dec" if "moe_gate_up_dec" in kern else "moe_gate_up_int"
    gu = kern.get(gu_name)
    roof = None
    if gu:
        # algorithmic bytes of one launch at b=1: gate + up rows of 2 experts,
        # plus the Q8_K activation row (4096 + 64 + 1024 B) and h out (2 x 14336 x 4 B)
        alg = 2 * 2 * PART + (4096 + 64 + 1024) + 2 * FF * 4
        ach = alg / (gu["avg_us"] * 1e-6) / 1e9
        tr = measured_traffic().get(gu_name) if S == 1 else None
        roof = {"bound": "hbm", "kernel": gu_name, "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4), "traffic": tr,
                "alg_bytes_per_launch": alg, "avg_us": gu["avg_us"],
                "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if tr else None}
    res = {
        "metric": "MoE-layer tokens/sec + % peak HBM GB/s, Mixtral-shape Q4_K decode b=1",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"mixtral-8x7b-moe-layer-q4k-decode-b{S}", "hidden": D, "expert_ffn": FF,
                   "experts": E, "top_k": K, "tokens_per_step": S, "weights": "Q4_K random-init blocks",
                   "layers_rotated": a.layers, "regime": ["avx2", "int8", "exact"][a.regime],
                   "launch": (f"hip-graph ({a.layers} layers per replay)" if graphs is not None else "eager")},
        "hbm_touched_GBps": round(touched / (ms_step * 1e-3) / 1e9, 1) if touched else None,
        "hbm_frac": round(touched / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4) if touched else None,
        "roofline": roof,
        "kernels_us": kern,
        "pcie_inclusive": pcie,
        "cpu_baseline": None,
    }
    if a.prefill_tokens > 0:
        res["prefill"] = prefill_leg(ctx, torch, a)
    legs = set() if a.no_extra else set(x for x in a.legs.split(",") if x)
    if "batches" in legs:
        res["decode_batches"] = [batch_leg(ctx, torch, a.layers, S2, rg) for S2 in (8, 32) for rg in (0, 1)]
    if "matvec_q4k" in legs:
        res["matvec_q4k"] = matvec_leg(ctx, torch, Q4_K, cpu_seconds=0.0 if a.no_cpu else a.cpu_seconds / 5,
                                       cpu_cap=a.cpu_threads)
    if "matvec_q6k" in legs:
        res["matvec_q6k"] = matvec_leg(ctx, torch, Q6_K)
    if "q4k_m" in legs:
        res["decode_b1_q4k_m"] = q4km_leg(ctx, torch)
    if "qwen3" in legs:
        res["qwen3"] = qwen3_leg(ctx, torch, cpu_seconds=0.0 if a.no_cpu else a.cpu_seconds / 4,
                                 cpu_cap=a.cpu_threads)
    if "c5_layer" in legs:
        res["c5_layer"] = c5_layer_leg(ctx, torch, cpu_seconds=0.0 if a.no_cpu else a.cpu_seconds / 4,
                                       cpu_cap=a.cpu_threads)
    if "preload" in legs:
        res["tier_preload"] = preload_leg(ctx, torch)
    if "decode_stack" in legs:
        res["decode_stack"] = decode_stack_leg(ctx, torch, MOE6B)
    if "c5_stack" in legs:
        res["c5_stack"] = decode_stack_leg(ctx, torch, DSV2LITE, cpu_seconds=0.0 if a.no_cpu else a.cpu_seconds,
                                           cpu_cap=a.cpu_threads)
    if "measure" in legs:  # the figures kestrel's planner would otherwise estimate (kmoe_measure)
        res["planner_inputs"] = {k: (round(v, 9) if isinstance(v, float) else v) for k, v in ctx.measure().items()}
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(ctx, torch, a.cpu_seconds, a.cpu_threads)
        if a.prefill_tokens > 0:
            res["prefill"]["cpu_baseline"] = cpu_prefill(ctx, a.prefill_tokens, a.cpu_seconds / 2, a.cpu_threads)
    print(json.dumps(res))
    ctx.close()


if __name__ == "__main__":
    main()
