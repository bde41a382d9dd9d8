"""Throughput of the quantized-linear hot path on one MI355X.

Primary line: FP8 e4m3 linear with dynamic per-tensor amax scaling, forward +
backward, over all four BERT-base linear shapes (768->768 x4 for Q/K/V/O,
768->3072, 3072->768) at 8192 tokens; x ~N(0,1) bf16 with 0.1% outliers x50,
W ~N(0,0.02). One step = fwd+bwd of the six linears. Value = algorithmic
TFLOP/s (3 GEMMs of 2*M*N*K per linear).

Secondary lines (same JSON object): the packed-INT4 + LoRA linear fwd+bwd at
the BERT-base FFN up-projection (x [4096, 768], W 768->3072, rank 16,
alpha 32) and the skinny-M inference sweep (M in {1,4,16,64} with group-64
scales and M in {1,16} with per-row scales, Qwen3-2B-shaped projections,
rank 32) with rotating weight copies larger than the 256 MB Infinity Cache.

The roofline object is for the dominant kernel (the fp8 MFMA GEMM): its
algorithmic FLOPs over its own launch durations, timed with HIP events on the
stream the kernels run on. cpu_baseline times the numpy oracle on host cores
on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0

BERT_LINEARS = [("q", 768, 768), ("k", 768, 768), ("v", 768, 768), ("o", 768, 768),
                ("ffn_up", 768, 3072), ("ffn_down", 3072, 768)]


def parse_args():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    # the GPU's clocks settle over the first ~50 replays of a 0.5 ms step
    # (measured: 0.480 ms over replays 6-55, 0.466 over later ones)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--tokens", type=int, default=8192)
    p.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=["fp8", "fp8delayed", "int4lora", "skinny", "bert", "qwen3",
                                      "fp8gemm", "copyref", "int4shapes", "vendor", "castref"],
                   default=None,
                   help="run one workload and nothing else (profiling); fp8gemm: three eager "
                        "launches of each fp8 GEMM call of one step; copyref: a plain 256 MiB "
                        "device copy, the reference for scaling FETCH_SIZE / WRITE_SIZE; "
                        "int4shapes: three eager INT4 + LoRA forwards and backwards at each "
                        "train-step linear shape (counter passes see eager launches only); "
                        "vendor: the fp8 GEMM calls and INT4 forwards next to hipBLASLt; castref: the "
                        "activation casts next to a plain copy of the same bytes")
    return p.parse_args()


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def bf16_tensor(a, device):
    import torch

    from oracle.codecs import f32_to_bf16_bits

    bits = f32_to_bf16_bits(np.asarray(a, np.float32)).view(np.int16)
    return torch.from_numpy(bits.copy()).to(device).view(torch.bfloat16)


def outlier_activations(g, m, k):
    x = g.standard_normal((m, k)).astype(np.float32)
    mask = g.random((m, k)) < 1e-3
    return np.where(mask, x * 50.0, x).astype(np.float32)


def time_region(fn, steps, warmup):
    """Mean ms per call of fn over `steps` calls after `warmup`, bracketed by
    device synchronization."""

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def maybe_graph(fn, use_graph):
    """Capture fn into a HIP graph (torch.cuda.CUDAGraph) when requested."""

    import torch

    if not use_graph:
        return fn, "eager"
    fn()  # first launch outside capture (one-time kernel attribute setup)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph.replay, "hipgraph"


def graph_time_per_call_ms(calls, replays=5):
    """GPU time per call of a batch of calls captured into one HIP graph
    (back-to-back on the device, no host launch gaps), HIP events around the
    replays on the capturing stream."""

    import torch

    for fn in calls[:2]:
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in calls:
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in calls:
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / (replays * len(calls))


# ---------------------------------------------------------------------------
# FP8 workload (primary)
# ---------------------------------------------------------------------------
def fp8_setup(tokens, device, seed=0):
    g = np.random.Generator(np.random.PCG64(seed))
    layers = []
    for name, k, n in BERT_LINEARS:
        x = bf16_tensor(outlier_activations(g, tokens, k), device)
        w = bf16_tensor(g.standard_normal((n, k)).astype(np.float32) * 0.02, device)
        gy = bf16_tensor(g.standard_normal((tokens, n)).astype(np.float32), device)
        layers.append((name, x, w, gy, k, n))
    return layers


def fp8_step_fn(layers):
    from representax_amd import ops

    def step():
        for _, x, w, gy, k, _ in layers:
            _, scales, codes = ops.fp8_linear_forward(x, w.t(), save_codes=True)
            ops.fp8_linear_backward_codes(codes, scales, gy, k=k, dtype=x.dtype,
                                          right_transposed=True)

    return step


def fp8_delayed_step_fn(layers, history_len=16):
    """The same step with delayed scaling: every operand is cast once with the
    scale its slot holds (saturating) while its amax is recorded (a linear's
    input and weight in one launch), and one launch updates all 18 slots'
    scales at the end of the step."""

    import torch

    from representax_amd import ops
    from representax_amd.precision import DelayedScaling

    dev = layers[0][1].device
    state = DelayedScaling(3 * len(layers), history_len, device=dev)
    slots = [state.allocate(("e4m3fn", "e4m3fn", "e5m2")) for _ in layers]
    sc = state.scales

    def step():
        for (_, x, w, gy, k, n), (sx, sw, sg) in zip(layers, slots):
            m = x.shape[0]
            (qx, _), (qw, qwt) = ops.fp8_cast_delayed2(x, sx, w, sw, state, "e4m3fn",
                                                       rowmajor=True, transposed=(False, True))
            ops._gemm_into(qx, "e4m3fn", sc[sx:sx + 1], qw, "e4m3fn", sc[sw:sw + 1],
                           torch.empty((m, n), dtype=x.dtype, device=dev))
            qg, _ = ops.fp8_cast_delayed(gy, state, sg, "e5m2", rowmajor=True)
            ops.fp8_linear_backward_gemms(qg, sc[sg:sg + 1], qx, sc[sx:sx + 1], qwt,
                                          sc[sw:sw + 1], k=k, dtype=x.dtype,
                                          right_transposed=True)
        state.update()

    return step


def run_fp8_delayed(layers, tokens, steps, warmup, use_graph):
    fn, mode = maybe_graph(fp8_delayed_step_fn(layers), use_graph)
    ms = time_region(fn, steps, warmup)
    return {
        "workload": "fp8 linear fwd+bwd, BERT-base shapes, 8192 tokens, delayed scaling (amax "
                    "history 16, saturating casts, one scale update per step; an extension, "
                    "not the reference's dynamic semantics)",
        "value": round(fp8_flops(tokens) / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4), "mode": mode,
    }


def fp8_flops(tokens):
    return sum(6.0 * tokens * k * n for _, k, n in BERT_LINEARS)


def fp8_gemm_calls(layers, paired=True):
    """The fp8 GEMM launches of one step on the codes and scales the step
    produces, with their algorithmic FLOPs and compulsory HBM bytes (fp8
    operands read once, bf16 outputs written once): per linear the forward
    product and the backward's input- and weight-gradient products. paired:
    the backward's two products as the step runs them, one
    fp8_linear_backward_gemms call (12 calls per step); otherwise each product
    alone (18 calls, for the per-product vendor comparison)."""

    import torch

    from representax_amd import ops

    calls = []
    for _, x, w, gy, k, n in layers:
        m = x.shape[0]
        s_x = ops.fp8_scale(x, "e4m3fn")
        s_w = ops.fp8_scale(w, "e4m3fn")
        s_g = ops.fp8_scale(gy, "e5m2")
        qx, qxt = ops.fp8_cast(x, s_x, "e4m3fn", rowmajor=True, transposed=True)
        qw, qwt = ops.fp8_cast(w, s_w, "e4m3fn", rowmajor=True, transposed=True)
        qg, qgt = ops.fp8_cast(gy, s_g, "e5m2", rowmajor=True, transposed=True)
        fwd_bytes = m * k + n * k + 2.0 * m * n
        dx_bytes = m * n + n * k + 2.0 * m * k
        dw_bytes = m * n + m * k + 2.0 * n * k
        calls.append((lambda a=qx, b=qw, sa=s_x, sb=s_w: ops.fp8_gemm(a, "e4m3fn", sa, b, "e4m3fn", sb),
                      2.0 * m * n * k, fwd_bytes))
        if paired:
            calls.append((lambda qg=qg, s_g=s_g, qx=qx, s_x=s_x, qwt=qwt, s_w=s_w, k=k:
                          ops.fp8_linear_backward_gemms(qg, s_g, qx, s_x, qwt, s_w, k=k,
                                                        dtype=torch.bfloat16,
                                                        right_transposed=True),
                          4.0 * m * n * k, dx_bytes + dw_bytes))
        else:
            calls.append((lambda a=qg, b=qwt, sa=s_g, sb=s_w: ops.fp8_gemm(a, "e5m2", sa, b, "e4m3fn", sb),
                          2.0 * m * n * k, dx_bytes))
            calls.append((lambda a=qgt, b=qxt, sa=s_x, sb=s_g: ops.fp8_gemm(a, "e5m2", sa, b, "e4m3fn", sb),
                          2.0 * m * n * k, dw_bytes))
    torch.cuda.synchronize()
    return calls


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "fp8_gemm_bert_shapes_hbm_traffic.md")


def profiled_traffic():
    """(HBM bytes per fp8 GEMM call, commit whose code they were measured on)
    from the committed --pmc summary (FETCH_SIZE and WRITE_SIZE of the 18
    calls, scaled by a plain copy's reading); (None, None) when the summary
    is absent. Counter passes cannot run inside the timed bench, so the
    figure is the summary's, tagged with its commit."""

    found = {}
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                for key in ("hbm_bytes_per_call", "measured_at_commit"):
                    if line.startswith(key + ":"):
                        found[key] = line.split(":", 1)[1].strip()
    except OSError:
        return None, None
    bytes_ = float(found["hbm_bytes_per_call"]) if "hbm_bytes_per_call" in found else None
    return bytes_, found.get("measured_at_commit")


def fp8_gemm_roofline(layers, rounds=4, reps=16):
    """Dominant kernels: the fp8 MFMA GEMM launches of one step (k_fp8_gemm
    for each forward, k_fp8_gemm_pair for each backward's two products, plus
    the split-K reduce where the weight gradient uses one). The 12 launches
    are captured in the step's order, `rounds` passes in one HIP graph, and
    timed with HIP events on the capturing stream, so each launch finds its
    operands as warm as in the step (each linear's codes are read once per
    pass), not left in the caches by the same launch before it; achieved =
    algorithmic FLOPs of the 12 launches / their time. For comparison each
    launch is also timed alone, `reps` times back to back
    (`avg_launch_us_repeated`)."""

    calls = fp8_gemm_calls(layers)
    fns = [fn for fn, _, _ in calls]
    total_ms = graph_time_per_call_ms(fns * rounds, replays=3) * len(calls)
    repeated_ms = sum(graph_time_per_call_ms([fn] * reps, replays=3) for fn in fns)
    total_flops = 0.0
    attainable_ms = 0.0
    for _, flops, nbytes in calls:
        total_flops += flops
        # the launch's own roofline, min(peak, AI x BW): 768 -> 768 products sit
        # below the fp8 ridge point (AI ~ 500 < 625 FLOP/B)
        attainable_ms += 1e3 * max(flops / (FP8_PEAK_TFLOPS * 1e12), nbytes / (HBM_PEAK_GBS * 1e9))
    achieved = total_flops / (total_ms * 1e-3) / 1e12
    traffic, traffic_commit = profiled_traffic()
    return {
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": FP8_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / FP8_PEAK_TFLOPS, 4),
        "frac_attainable": round(attainable_ms / total_ms, 4),
        "traffic": traffic,
        "traffic_source": {"profile": os.path.relpath(TRAFFIC_PROFILE, ROOT),
                           "measured_at_commit": traffic_commit},
        "kernel": "k_fp8_gemm (forward, e4m3xe4m3) and k_fp8_gemm_pair (backward dX and dW, "
                  "e5m2xe4m3, in one launch; + k_fp8_split_reduce where dW is split-K); 12 calls "
                  "per step",
        "timing": f"the 12 launches in step order, {rounds} passes per HIP graph",
        "avg_launch_us": round(1e3 * total_ms / len(calls), 2),
        "avg_launch_us_repeated": round(1e3 * repeated_ms / len(calls), 2),
        "flops_per_launch_avg": total_flops / len(calls),
        "algorithmic_bytes_per_launch_avg": fp8_gemm_bytes(layers) / len(calls),
        "gemm_us_per_step": round(1e3 * total_ms, 1),
    }


def fp8_quantize_report(layers, step_ms, gemm_us):
    """The dynamic quantize passes of one step (amax, then the cast) against
    HBM bandwidth. Their time is the step's minus its 12 GEMM launches' (each
    timed alone in a graph); their algorithmic bytes per linear are
    5 MK + 6 NK + 5 MN: the amax pass reads x, W and g in bf16, the cast reads
    them again and writes one byte per element of x and g (row-major; the
    weight gradient reads them along the tokens) and two of W (row-major for
    the forward, transposed for the input gradient)."""

    nbytes = 0.0
    for _, x, _, _, k, n in layers:
        m = x.shape[0]
        nbytes += 5.0 * m * k + 6.0 * n * k + 5.0 * m * n
    us = 1e3 * step_ms - gemm_us
    gbs = nbytes / (us * 1e-6) / 1e9 if us > 0 else None
    return {"us_per_step": round(us, 1), "algorithmic_bytes_per_step": nbytes,
            "gbs": None if gbs is None else round(gbs, 1),
            "frac_hbm": None if gbs is None else round(gbs / HBM_PEAK_GBS, 4),
            "kernels": "k_amax_tiles + k_fp8_cast_tile (12 each per step)",
            "timing": "step time minus the 12 GEMM launches' graph-timed time"}


def fp8_gemm_bytes(layers):
    """Compulsory HBM bytes of the step's GEMM products: fp8 operands read
    once, the bf16 outputs (y, dX, dW) written once."""

    total = 0.0
    for _, x, _, _, k, n in layers:
        m = x.shape[0]
        total += m * k + n * k + m * n * 2          # forward: x, W codes; y bf16
        total += m * n + n * k + m * k * 2          # dX: g, W^T codes; dX bf16
        total += m * n + m * k + n * k * 2          # dW: g^T, x^T codes; dW bf16
    return total


def run_fp8gemm_only(layers):
    import torch

    for fn, _, _ in fp8_gemm_calls(layers):
        for _ in range(3):
            fn()
    torch.cuda.synchronize()


INT4_STEP_SHAPES = [("bert q/k/v/o", 32768, 768, 768, 16), ("bert ffn up", 32768, 768, 3072, 16),
                    ("bert ffn down", 32768, 3072, 768, 16), ("qwen3 q/o", 16384, 2048, 2048, 32),
                    ("qwen3 gate/up", 16384, 2048, 6144, 32), ("qwen3 down", 16384, 6144, 2048, 32)]


def run_int4_shapes(reps=3, group=64):
    """Eager INT4 + LoRA forward and backward calls at every linear shape of
    the BERT-base and Qwen3-2B-shaped steps (group 64), for counter passes."""

    import torch

    from representax_amd import ops

    dev = torch.device("cuda:0")
    g = np.random.Generator(np.random.PCG64(9))
    out = []
    for name, m, k, n, r in INT4_STEP_SHAPES:
        x = bf16_tensor(g.standard_normal((m, k)).astype(np.float32), dev)
        gy = bf16_tensor(g.standard_normal((m, n)).astype(np.float32), dev)
        w = torch.from_numpy((g.standard_normal((n, k)) * 0.02).astype(np.float32)).to(dev)
        packed, scales = ops.int4_pack(w, group)
        a = bf16_tensor(g.standard_normal((r, k)).astype(np.float32) * 0.02, dev)
        b = bf16_tensor(g.standard_normal((n, r)).astype(np.float32) * 0.02, dev)
        for _ in range(reps):
            _, h = ops.int4lora_forward(x, packed, scales, a, b, scaling=2.0, group_size=group)
            ops.int4lora_backward(gy, x, packed, scales, a, b, h, scaling=2.0, group_size=group)
        torch.cuda.synchronize()
        out.append(name)
        del x, gy, w
        torch.cuda.empty_cache()
    print(json.dumps({"int4_shapes": out, "reps": reps}))


def run_vendor(layers):
    """The platform library on the same products, for comparison: every fp8
    GEMM call of the BERT-base step against torch._scaled_mm (hipBLASLt,
    e4m3 x e4m3 with scalar scales, bf16 out), and the INT4 + LoRA forward at
    the train-step linear shapes against a plain bf16 torch.matmul (hipBLASLt)
    of the same M, K, N without the adapter. GPU time per call inside a HIP
    graph of 16 calls, as for the roofline."""

    import torch

    from representax_amd import ops

    dev = torch.device("cuda:0")
    names = []
    for nm, k, n in BERT_LINEARS:
        names += [(f"{nm} fwd", 8192, n, k), (f"{nm} dX", 8192, k, n), (f"{nm} dW", n, k, 8192)]
    fp8 = []
    for (fn, _, _), (nm, m, n, k) in zip(fp8_gemm_calls(layers, paired=False), names):
        ours = graph_time_per_call_ms([fn] * 16, replays=3) * 1e3
        a = torch.randn(m, k, device=dev).to(torch.float8_e4m3fn)
        b = torch.randn(n, k, device=dev).to(torch.float8_e4m3fn)
        one = torch.tensor(1.0, device=dev)
        lib = graph_time_per_call_ms(
            [lambda: torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)]
            * 16, replays=3) * 1e3
        fp8.append({"call": nm, "m": m, "n": n, "k": k, "ours_us": round(ours, 2),
                    "hipblaslt_us": round(lib, 2)})
        del a, b
    g = np.random.Generator(np.random.PCG64(3))
    int4 = []
    for name, m, k, n, r in INT4_STEP_SHAPES:
        x = bf16_tensor(g.standard_normal((m, k)).astype(np.float32), dev)
        w = torch.from_numpy((g.standard_normal((n, k)) * 0.02).astype(np.float32)).to(dev)
        packed, scales = ops.int4_pack(w, 64)
        a = bf16_tensor(g.standard_normal((r, k)).astype(np.float32) * 0.02, dev)
        b = bf16_tensor(g.standard_normal((n, r)).astype(np.float32) * 0.02, dev)
        wt = w.to(torch.bfloat16).t().contiguous()
        ours = graph_time_per_call_ms(
            [lambda: ops.int4lora_forward(x, packed, scales, a, b, scaling=2.0, group_size=64)] * 16,
            replays=3) * 1e3
        lib = graph_time_per_call_ms([lambda: torch.matmul(x, wt)] * 16, replays=3) * 1e3
        int4.append({"linear": name, "m": m, "k": k, "n": n, "rank": r,
                     "int4lora_fwd_us": round(ours, 2), "bf16_matmul_us": round(lib, 2)})
        del x, w, packed, scales, a, b, wt
        torch.cuda.empty_cache()
    print(json.dumps({"fp8_gemm_calls": fp8,
                      "fp8_total_us": {"ours": round(sum(c["ours_us"] for c in fp8), 1),
                                       "hipblaslt": round(sum(c["hipblaslt_us"] for c in fp8), 1)},
                      "int4lora_forward_vs_bf16": int4}))


def run_castref(layers, reps=16):
    """The dynamic cast of each distinct BERT-base activation shape (8192 x 768
    and 8192 x 3072 bf16 -> e4m3 codes in both layouts, the scale given)
    against a plain device copy that moves the same bytes (a bf16 tensor of
    the same shape: 2 bytes read and 2 written per element, as the cast
    reads 2 and writes 1 + 1). GPU time per call in a HIP graph of `reps`."""

    import torch

    from representax_amd import ops

    out = []
    for name, x, _, _, k, _ in (layers[0], layers[5]):
        s = ops.fp8_scale(x, "e4m3fn")
        cast = graph_time_per_call_ms(
            [lambda: ops.fp8_cast(x, s, "e4m3fn", rowmajor=True, transposed=True)] * reps,
            replays=3) * 1e3
        dst = torch.empty_like(x)
        copy = graph_time_per_call_ms([lambda: dst.copy_(x)] * reps, replays=3) * 1e3
        out.append({"tensor": f"{x.shape[0]} x {k} bf16", "cast_both_layouts_us": round(cast, 2),
                    "copy_same_bytes_us": round(copy, 2), "ratio": round(cast / copy, 3)})
    print(json.dumps({"castref": out}))


def run_copyref(nbytes=256 << 20):
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copyref_bytes_each_way": nbytes, "launches": 3}))


def host_threads():
    """(threads the numpy baseline uses, CPUs this process may run on, CPU
    model): BLAS runs OMP_NUM_THREADS threads, capped by the affinity mask."""

    allowed = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(allowed, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else allowed
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return threads, allowed, model


def fp8_cpu_baseline(seed=1):
    """Oracle fp8 linear fwd+bwd (numpy, float32 BLAS accumulate) on a bounded
    sample: the 768->3072 linear at 1024 tokens, repeated to ~10-20 s."""

    from oracle import fp8 as ofp8
    from oracle.codecs import bf16_round

    g = np.random.Generator(np.random.PCG64(seed))
    m, k, n = 1024, 768, 3072
    x = bf16_round(outlier_activations(g, m, k))
    w = bf16_round(g.standard_normal((n, k)).astype(np.float32) * 0.02)
    gy = bf16_round(g.standard_normal((m, n)).astype(np.float32))
    flops = 6.0 * m * n * k
    reps = 0
    t0 = time.perf_counter()
    while True:
        ofp8.fp8_linear_forward(x, w.T, acc=np.float32)
        ofp8.fp8_linear_backward(x, w.T, gy, acc=np.float32)
        reps += 1
        if time.perf_counter() - t0 > 10.0 or reps >= 50:
            break
    dt = (time.perf_counter() - t0) / reps
    threads, allowed, model = host_threads()
    return {
        "value": round(flops / dt / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"numpy oracle fp8 linear fwd+bwd, 768->3072 at {m} tokens, {reps} reps, "
                  f"{dt * 1e3:.0f} ms each (fp32 BLAS accumulate); {threads} BLAS threads of "
                  f"{allowed} allowed CPUs, {model}",
    }


def int4lora_cpu_baseline(group_size=None, seed=3):
    """Oracle INT4 + LoRA linear fwd+bwd (numpy, float32 BLAS accumulate) on
    a bounded sample of the config: 512 of the 4096 tokens, 768->3072,
    rank 16, alpha 32, repeated to ~10 s."""

    from oracle import int4 as oint4
    from oracle import lora as olora
    from oracle.codecs import bf16_round

    g = np.random.Generator(np.random.PCG64(seed))
    m, k, n, r = 512, 768, 3072, 16
    x = bf16_round(g.standard_normal((m, k)).astype(np.float32))
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = (g.standard_normal((r, k)) * 0.02).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.02).astype(np.float32)
    gy = bf16_round(g.standard_normal((m, n)).astype(np.float32))
    packed, scales = oint4.pack_int4(w, group_size)
    flops = 2 * m * n * k + 2 * m * k * r + 2 * m * r * n + 2 * m * n * k + 4 * m * n * r + 4 * m * r * k
    reps = 0
    t0 = time.perf_counter()
    while True:
        _, h = olora.lora_forward(x, packed, scales, a, b, alpha=32.0, rank=r,
                                  group_size=group_size, acc=np.float32)
        olora.lora_backward(gy, x, packed, scales, a, b, h, alpha=32.0, rank=r,
                            group_size=group_size, acc=np.float32)
        reps += 1
        if time.perf_counter() - t0 > 10.0 or reps >= 50:
            break
    dt = (time.perf_counter() - t0) / reps
    threads, allowed, model = host_threads()
    scales_kind = "per-row" if group_size is None else f"group {group_size}"
    return {
        "value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"numpy oracle INT4-LoRA fwd+bwd ({scales_kind} scales, dequant included), "
                  f"768->3072 r16 at {m} of the 4096 tokens, {reps} reps, {dt * 1e3:.0f} ms each; "
                  f"{threads} BLAS threads of {allowed} allowed CPUs, {model}",
    }


def skinny_cpu_baseline(seed=4):
    """Oracle skinny-M forward (numpy, float32 BLAS accumulate, dequant
    included) at M = 1 on the 2048->6144 projection, group 64, rank 32."""

    from oracle import int4 as oint4
    from oracle import lora as olora
    from oracle.codecs import bf16_round

    g = np.random.Generator(np.random.PCG64(seed))
    m, k, n, r, group = 1, 2048, 6144, 32, 64
    x = bf16_round(g.standard_normal((m, k)).astype(np.float32))
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = (g.standard_normal((r, k)) * 0.02).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.02).astype(np.float32)
    packed, scales = oint4.pack_int4(w, group)
    nbytes = n * k / 2 + n * (k // group) * 2 + (r * k + n * r) * 2 + m * k * 2 + m * n * 2
    reps = 0
    t0 = time.perf_counter()
    while True:
        olora.lora_forward(x, packed, scales, a, b, alpha=64.0, rank=r, group_size=group,
                           acc=np.float32)
        reps += 1
        if time.perf_counter() - t0 > 10.0 or reps >= 200:
            break
    dt = (time.perf_counter() - t0) / reps
    threads, allowed, model = host_threads()
    return {
        "value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "us_per_call": round(dt * 1e6, 1),
        "sample": f"numpy oracle INT4-LoRA forward (dequant included), M=1, 2048->6144, group 64, "
                  f"r32, {reps} reps; {threads} BLAS threads of {allowed} allowed CPUs, {model}",
    }


# ---------------------------------------------------------------------------
# INT4 + LoRA workload (secondary)
# ---------------------------------------------------------------------------
def int4lora_setup(device, group_size=None, seed=2):
    import torch

    from representax_amd import ops

    g = np.random.Generator(np.random.PCG64(seed))
    m, k, n, r = 4096, 768, 3072, 16
    x = bf16_tensor(g.standard_normal((m, k)).astype(np.float32), device)
    w = torch.from_numpy((g.standard_normal((n, k)) * 0.02).astype(np.float32)).to(device)
    packed, scales = ops.int4_pack(w, group_size)
    a = bf16_tensor(g.standard_normal((r, k)).astype(np.float32) * 0.02, device)
    b = bf16_tensor(g.standard_normal((n, r)).astype(np.float32) * 0.02, device)
    bias = bf16_tensor(np.zeros(n, np.float32), device).view(torch.uint16)
    gy = bf16_tensor(g.standard_normal((m, n)).astype(np.float32), device)
    return dict(x=x, packed=packed, scales=scales, a=a, b=b, bias=bias, gy=gy, m=m, k=k, n=n, r=r,
                group=group_size)


def int4lora_step_fn(c):
    from representax_amd import ops

    def step():
        _, h = ops.int4lora_forward(c["x"], c["packed"], c["scales"], c["a"], c["b"], scaling=2.0,
                                    group_size=c["group"], bias_bits=c["bias"])
        ops.int4lora_backward(c["gy"], c["x"], c["packed"], c["scales"], c["a"], c["b"], h,
                              scaling=2.0, group_size=c["group"])

    return step


def int4lora_flops(c):
    m, k, n, r = c["m"], c["k"], c["n"], c["r"]
    fwd = 2 * m * n * k + 2 * m * k * r + 2 * m * r * n
    bwd = 2 * m * n * k + 4 * m * n * r + 4 * m * r * k
    return float(fwd + bwd)


def int4lora_roofline(c, reps=20):
    """The fused dequant + MFMA forward GEMM (the path's defining kernel)."""

    from representax_amd import ops

    def fwd():
        ops.int4lora_forward(c["x"], c["packed"], c["scales"], c["a"], c["b"], scaling=2.0,
                             group_size=c["group"], bias_bits=c["bias"])

    ms = graph_time_per_call_ms([fwd] * reps)
    m, k, n, r = c["m"], c["k"], c["n"], c["r"]
    flops = 2.0 * m * n * k + 2 * m * k * r + 2 * m * r * n
    achieved = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "kernel": "int4lora_forward (rank-r down kernel + fused dequant GEMM)",
            "avg_call_us": round(ms * 1e3, 2), "dequant": int4_dequant_rate(c, reps)}


def int4_dequant_rate(c, reps=20):
    """The dequantization stage on its own: the config's packed weight to a
    bf16 [N, K] matrix (rpx_int4_dequant, bit-exact bf16(q * s)), the same
    unpack the GEMM applies to its B tiles in LDS. Algorithmic bytes: packed
    codes and scales read once, the bf16 weight written once."""

    from representax_amd import ops

    n, k = c["n"], c["k"]

    def deq():
        ops.int4_dequant(c["packed"], c["scales"], k, c["group"])

    ms = graph_time_per_call_ms([deq] * reps)
    nbytes = float(c["packed"].numel() + 2 * c["scales"].numel() + 2 * n * k)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": "k_int4_dequant (rpx_int4_dequant)", "us_per_call": round(ms * 1e3, 2),
            "algorithmic_bytes": nbytes, "gbs": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def run_int4lora(steps, warmup, use_graph, group_size=None):
    import torch

    c = int4lora_setup(torch.device("cuda:0"), group_size)
    fn, mode = maybe_graph(int4lora_step_fn(c), use_graph)
    ms = time_region(fn, steps, warmup)
    tflops = int4lora_flops(c) / (ms * 1e-3) / 1e12
    line = {
        "workload": "int4lora linear fwd+bwd, x[4096,768] bf16, W 768->3072 INT4 "
                    f"({'per-row scales' if group_size is None else f'group {group_size}'}), "
                    "rank 16, alpha 32",
        "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "mode": mode,
        "roofline": int4lora_roofline(c),
    }
    return line


# ---------------------------------------------------------------------------
# Skinny-M inference sweep (secondary)
# ---------------------------------------------------------------------------
SKINNY_SHAPES = [(2048, 6144), (6144, 2048), (2048, 2048)]


def linear_rooflines(shapes, tokens, group, rank, reps=10, seed=8):
    """Each distinct INT4 + LoRA linear of a train step at its step size:
    forward and backward GPU time per call inside a HIP graph of `reps`
    calls, TFLOP/s of the algorithmic work (fwd 2MNK + 2MKr + 2MrN, bwd
    2MNK + 4MNr + 4MrK) and its fraction of the bf16 dense peak. `shapes`
    holds (name, K, N, calls per layer)."""

    import torch

    from representax_amd import ops

    dev = torch.device("cuda:0")
    g = np.random.Generator(np.random.PCG64(seed))
    k_max = max(k for _, k, _, _ in shapes)
    n_max = max(n for _, _, n, _ in shapes)
    x0 = bf16_tensor(g.standard_normal((tokens, k_max)).astype(np.float32), dev)
    gy0 = bf16_tensor(g.standard_normal((tokens, n_max)).astype(np.float32), dev)
    out = []
    for name, k, n, count in shapes:
        w = torch.from_numpy((g.standard_normal((n, k)) * 0.02).astype(np.float32)).to(dev)
        packed, scales = ops.int4_pack(w, group)
        a = bf16_tensor(g.standard_normal((rank, k)).astype(np.float32) * 0.02, dev)
        b = bf16_tensor(g.standard_normal((n, rank)).astype(np.float32) * 0.02, dev)
        x = x0[:, :k].contiguous()
        gy = gy0[:, :n].contiguous()
        _, h = ops.int4lora_forward(x, packed, scales, a, b, scaling=2.0, group_size=group)

        def fwd():
            ops.int4lora_forward(x, packed, scales, a, b, scaling=2.0, group_size=group)

        def bwd():
            ops.int4lora_backward(gy, x, packed, scales, a, b, h, scaling=2.0, group_size=group)

        f_ms = graph_time_per_call_ms([fwd] * reps, replays=3)
        b_ms = graph_time_per_call_ms([bwd] * reps, replays=3)
        m = tokens
        f_fl = 2.0 * m * n * k + 2 * m * k * rank + 2 * m * rank * n
        b_fl = 2.0 * m * n * k + 4 * m * n * rank + 4 * m * rank * k
        f_tf = f_fl / (f_ms * 1e-3) / 1e12
        b_tf = b_fl / (b_ms * 1e-3) / 1e12
        out.append({"linear": name, "per_layer": count, "k": k, "n": n,
                    "fwd_us": round(f_ms * 1e3, 1), "fwd_tflops": round(f_tf, 1),
                    "fwd_frac": round(f_tf / BF16_PEAK_TFLOPS, 4),
                    "bwd_us": round(b_ms * 1e3, 1), "bwd_tflops": round(b_tf, 1),
                    "bwd_frac": round(b_tf / BF16_PEAK_TFLOPS, 4),
                    "_flops": (f_fl, b_fl)})
        del w, packed, scales, a, b, x, gy, h
    del x0, gy0
    torch.cuda.empty_cache()
    return out


BERT_STEP_LINEARS = (("q/k/v/o", 768, 768, 4), ("ffn up", 768, 3072, 1),
                     ("ffn down", 3072, 768, 1))
QWEN3_STEP_LINEARS = (("q/o", 2048, 2048, 2), ("k/v", 2048, 1024, 2),
                      ("gate/up", 2048, 6144, 2), ("down", 6144, 2048, 1))


def step_linear_roofline(per_linear, remat):
    """The step's INT4 + LoRA linears as one roofline entry: their
    algorithmic FLOPs over their measured per-call times, weighted by the
    step's call mix (per layer: each linear's forward once, again under full
    rematerialization, and its backward once)."""

    fwd_calls = 2 if remat == "full" else 1
    flops = sum(p["per_layer"] * (fwd_calls * p["_flops"][0] + p["_flops"][1]) for p in per_linear)
    us = sum(p["per_layer"] * (fwd_calls * p["fwd_us"] + p["bwd_us"]) for p in per_linear)
    achieved = flops / (us * 1e-6) / 1e12
    for p in per_linear:
        p.pop("_flops", None)
    return {
        "bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None,
        "kernel": "INT4-LoRA linear fwd+bwd (fused dequant MFMA GEMM + rank-r kernels; dx "
                  "GEMM + dA/dB), each distinct linear timed per call in HIP graphs of 10 calls "
                  f"at the step's token count, weighted by the step's calls per layer ({fwd_calls} "
                  "forward(s) and one backward each)",
        "per_linear": per_linear,
    }


def bert_linear_rooflines(tokens=32768, group=64, rank=16, reps=10):
    return linear_rooflines(BERT_STEP_LINEARS, tokens, group, rank, reps)


def qwen3_linear_rooflines(tokens=16384, group=64, rank=32, reps=10):
    return linear_rooflines(QWEN3_STEP_LINEARS, tokens, group, rank, reps)


def trainstep_cpu_baseline(shapes, layers, rank, group, sample_tokens, remat="full", seed=5,
                           budget_s=10.0):
    """Oracle INT4 + LoRA fwd+bwd (numpy, float32 BLAS accumulate, dequant
    included) of one layer's linears at `sample_tokens` tokens, repeated to
    about `budget_s` seconds, scaled to the step's linear work per token:
    `layers` layers, each linear's forward twice under full remat and its
    backward once. Attention, norms, the loss and the optimizer are left out,
    so the figure bounds the CPU's tokens/s from above."""

    from oracle import int4 as oint4
    from oracle import lora as olora
    from oracle.codecs import bf16_round

    g = np.random.Generator(np.random.PCG64(seed))
    m = sample_tokens
    cases = []
    for _, k, n, count in shapes:
        x = bf16_round(g.standard_normal((m, k)).astype(np.float32))
        w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
        a = (g.standard_normal((rank, k)) * 0.02).astype(np.float32)
        b = (g.standard_normal((n, rank)) * 0.02).astype(np.float32)
        gy = bf16_round(g.standard_normal((m, n)).astype(np.float32))
        packed, scales = oint4.pack_int4(w, group)
        cases.append((count, x, packed, scales, a, b, gy))
    fwd_calls = 2 if remat == "full" else 1
    t_layer = 0.0
    reps = 0
    t0 = time.perf_counter()
    while True:
        t_rep = 0.0
        for count, x, packed, scales, a, b, gy in cases:
            t1 = time.perf_counter()
            _, h = olora.lora_forward(x, packed, scales, a, b, alpha=2.0 * rank, rank=rank,
                                      group_size=group, acc=np.float32)
            t2 = time.perf_counter()
            olora.lora_backward(gy, x, packed, scales, a, b, h, alpha=2.0 * rank, rank=rank,
                                group_size=group, acc=np.float32)
            t3 = time.perf_counter()
            t_rep += count * (fwd_calls * (t2 - t1) + (t3 - t2))
        t_layer += t_rep
        reps += 1
        if time.perf_counter() - t0 > budget_s or reps >= 20:
            break
    t_layer /= reps
    flops = sum(count * (fwd_calls * (2.0 * m * n * k + 2 * m * k * rank + 2 * m * rank * n)
                         + 2.0 * m * n * k + 4 * m * n * rank + 4 * m * rank * k)
                for (_, k, n, count) in shapes) * layers
    step_s = t_layer * layers
    threads, allowed, model = host_threads()
    names = ", ".join(f"{name} {k}->{n} x{count}" for name, k, n, count in shapes)
    return {
        "value": round(m / step_s, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
        "tflops": round(flops / step_s / 1e12, 5),
        "sample": f"numpy oracle INT4-LoRA fwd+bwd of one layer's linears ({names}; group "
                  f"{group}, r{rank}, dequant included) at {m} tokens, {reps} reps, "
                  f"{t_layer * 1e3:.0f} ms per layer with {fwd_calls} forward(s) + 1 backward "
                  f"per linear, scaled to {layers} layers; linears only (no attention, norms, "
                  f"loss or optimizer), so an upper bound on the CPU's tokens/s; {threads} BLAS "
                  f"threads of {allowed} allowed CPUs, {model}",
    }


def run_bert(steps=10, warmup=3, remat="full"):
    """BERT-base encoder train step with every Q/K/V/O/FFN linear packed INT4
    (group 64) + rank-16 LoRA (alpha 32): in-batch MNR loss over 64
    query/document pairs x 256 tokens, bf16 compute, per-layer
    rematerialization (the reference's default, full), global-norm clipping
    at 1.0 and the non-finite step guard, AdamW on the fp32 LoRA masters, the
    whole step replayed as one HIP graph."""

    import torch

    from representax_amd.trainstep import BertConfig, MNRTrainStep, build_int4lora_encoder

    cfg = BertConfig()
    pairs, seq = 64, 256
    model = build_int4lora_encoder(cfg, rank=16, alpha=32.0, group_size=64, seed=0,
                                   device=torch.device("cuda:0"))
    step = MNRTrainStep(model, batch=pairs, sequence=seq, remat=remat)
    step.capture(warmup=2)
    ms = time_region(step, steps, warmup)
    loss = float(step.loss)
    tokens = 2 * pairs * seq
    flops = cfg.step_flops(2 * pairs, seq, remat=remat == "full")
    recompute = "full per-layer rematerialization" if remat == "full" else "no recompute"
    line = {
        "workload": "BERT-base (12L, H768, 12 heads, FFN 3072, vocab 30522) train step, every "
                    "Q/K/V/O/FFN linear INT4 group-64 + LoRA r16 a32, in-batch MNR loss (scale 20), "
                    "64 query/document pairs x 256 tokens, bf16 compute, AdamW on fp32 LoRA "
                    f"masters, max grad norm 1.0, non-finite step guard, {recompute}, HIP graph",
        "remat": remat,
        "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s",
        "ms_per_step": round(ms, 3), "tokens_per_step": tokens,
        "matrix_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "matrix_tflop_per_step": round(flops / 1e12, 3),
        "loss_after_timed_steps": round(loss, 4),
        "grad_norm_last_step": round(float(step.grad_norm), 4),
    }
    del step, model
    torch.cuda.empty_cache()
    return line


def run_qwen3(steps=6, warmup=2, remat="full"):
    """Qwen3-VL-2B-shaped text tower train step (28 layers, hidden 2048, 16 Q /
    8 KV heads of 128, SwiGLU 6144, vocab 151936) with all seven projections
    INT4 group 64 + LoRA r32 (alpha 64): last-token-pooled MNR loss over 16
    query/document pairs x 512 tokens, bf16 compute, per-layer
    rematerialization (full, the reference's default), global-norm clipping
    at 1.0 and the non-finite step guard, AdamW on the fp32 LoRA masters, one
    HIP graph per step."""

    import torch

    from representax_amd.trainstep import MNRTrainStep, Qwen3TextConfig, build_int4lora_qwen3

    cfg = Qwen3TextConfig()
    pairs, seq = 16, 512
    model = build_int4lora_qwen3(cfg, rank=32, alpha=64.0, group_size=64, seed=0,
                                 device=torch.device("cuda:0"))
    step = MNRTrainStep(model, batch=pairs, sequence=seq, remat=remat)
    step.capture(warmup=2)
    ms = time_region(step, steps, warmup)
    tokens = 2 * pairs * seq
    flops = cfg.step_flops(2 * pairs, seq, remat=remat == "full")
    recompute = "full per-layer rematerialization" if remat == "full" else "no recompute"
    line = {
        "workload": "Qwen3-VL-2B-shaped text tower train step (28L, H2048, 16 Q / 8 KV heads x 128, "
                    "SwiGLU 6144, vocab 151936), all 7 projections INT4 group-64 + LoRA r32 a64, "
                    "last-token MNR loss, 16 query/document pairs x 512 tokens, bf16 compute, AdamW "
                    f"on fp32 LoRA masters, max grad norm 1.0, non-finite step guard, {recompute}, "
                    "HIP graph",
        "remat": remat,
        "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s",
        "ms_per_step": round(ms, 3), "tokens_per_step": tokens,
        "matrix_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "matrix_tflop_per_step": round(flops / 1e12, 3),
        "loss_after_timed_steps": round(float(step.loss), 4),
        "grad_norm_last_step": round(float(step.grad_norm), 4),
    }
    del step, model
    torch.cuda.empty_cache()
    return line


def run_skinny(batch=96, latency_calls=64):
    """Skinny-M INT4 + LoRA r32 forward on the Qwen3-2B projection shapes:
    group-64 scales at M in {1, 4, 16, 64}, and the reference's per-row
    scales at M in {1, 16}. `us_per_call`: GPU time per call inside a HIP
    graph of `batch` calls that cycle through a pool of weight copies larger
    than the 256 MB Infinity Cache, so every call streams its packed weight
    from HBM. `p50_us`: median over `latency_calls` single eager calls (HIP
    events around each, weights cycling the same way). Every call is the
    inference form (``need_h=False``: h stays in the call's scratch, y is the
    one output). HBM bytes: packed weight, scales, A, B, x and y."""

    import torch

    from representax_amd import ops

    dev = torch.device("cuda:0")
    g = np.random.Generator(np.random.PCG64(5))
    r = 32
    out = []
    for group, ms in ((64, (1, 4, 16, 64)), (None, (1, 16))):
        for k, n in SKINNY_SHAPES:
            n_groups = 1 if group is None else k // group
            per_copy = n * k // 2 + n * n_groups * 2 + (r * k + n * r) * 2
            copies = max(8, int(np.ceil(300e6 / per_copy)))
            w = torch.from_numpy((g.standard_normal((n, k)) * 0.02).astype(np.float32)).to(dev)
            packed, scales = ops.int4_pack(w, group_size=group)
            del w
            a0 = bf16_tensor(g.standard_normal((r, k)).astype(np.float32) * 0.02, dev)
            b0 = bf16_tensor(g.standard_normal((n, r)).astype(np.float32) * 0.02, dev)
            pool = [(packed.clone(), scales.clone(), a0.clone(), b0.clone()) for _ in range(copies)]
            for m in ms:
                x = bf16_tensor(g.standard_normal((m, k)).astype(np.float32), dev)
                calls = []
                for i in range(batch):
                    p, s, a, b = pool[i % copies]
                    calls.append(lambda p=p, s=s, a=a, b=b: ops.int4lora_forward(
                        x, p, s, a, b, scaling=2.0, group_size=group, need_h=False))
                us = graph_time_per_call_ms(calls, replays=3) * 1e3
                lat = []
                for i in range(latency_calls):
                    fn = calls[(i * 7) % batch]
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    fn()
                    e1.record()
                    e1.synchronize()
                    lat.append(e0.elapsed_time(e1) * 1e3)
                nbytes = n * k / 2 + n * n_groups * 2 + (r * k + n * r) * 2 + m * k * 2 + m * n * 2
                out.append({"m": m, "k": k, "n": n, "group": group, "us_per_call": round(us, 2),
                            "p50_us": round(float(np.median(lat)), 2),
                            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                            "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
            del pool
            torch.cuda.empty_cache()
    return {"workload": "skinny-M INT4 + LoRA r32 forward, Qwen3-2B projection shapes, group-64 "
                        "and per-row scales; us_per_call inside a HIP graph of 96 calls cycling "
                        "weight copies > 256 MB, p50_us over single eager calls", "points": out,
            "shared_input": run_skinny_shared(batch, latency_calls)}


SHARED_INPUT_GROUPS = [("qwen3 q/k/v", 2048, (2048, 1024, 1024)),
                       ("qwen3 gate/up", 2048, (6144, 6144))]


def run_skinny_shared(batch=96, latency_calls=64, group=64, r=32):
    """Projections of one input (the Qwen3-2B tower's q/k/v and gate/up) at
    M in {1, 4}: one rpx_int4lora_forward_multi call against one call per
    projection, both per call inside a HIP graph of `batch` calls cycling
    weight copies beyond the MALL, plus the multi call's eager p50 (inference
    form, ``need_h=False``, as the model's shared-input path calls it). HBM bytes:
    every projection's packed weight, scales, A, B and y, and x once."""

    import torch

    from representax_amd import ops

    dev = torch.device("cuda:0")
    g = np.random.Generator(np.random.PCG64(6))
    out = []
    for name, k, ns in SHARED_INPUT_GROUPS:
        per_copy = sum(n * k // 2 + n * (k // group) * 2 + (r * k + n * r) * 2 for n in ns)
        copies = max(8, int(np.ceil(300e6 / per_copy)))
        base = []
        for n in ns:
            w = torch.from_numpy((g.standard_normal((n, k)) * 0.02).astype(np.float32)).to(dev)
            packed, scales = ops.int4_pack(w, group_size=group)
            a = bf16_tensor(g.standard_normal((r, k)).astype(np.float32) * 0.02, dev)
            b = bf16_tensor(g.standard_normal((n, r)).astype(np.float32) * 0.02, dev)
            base.append((packed, scales, a, b))
        pool = [[tuple(t.clone() for t in p) for p in base] for _ in range(copies)]
        for m in (1, 4):
            x = bf16_tensor(g.standard_normal((m, k)).astype(np.float32), dev)
            multi, separate = [], []
            for i in range(batch):
                projs = pool[i % copies]
                multi.append(lambda projs=projs: ops.int4lora_forward_multi(
                    x, [(p, s, a, b, 2.0, group, None) for p, s, a, b in projs], need_h=False))
                separate.append(lambda projs=projs: [
                    ops.int4lora_forward(x, p, s, a, b, scaling=2.0, group_size=group,
                                         need_h=False)
                    for p, s, a, b in projs])
            us_multi = graph_time_per_call_ms(multi, replays=3) * 1e3
            us_sep = graph_time_per_call_ms(separate, replays=3) * 1e3
            lat = []
            for i in range(latency_calls):
                fn = multi[(i * 7) % batch]
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                fn()
                e1.record()
                e1.synchronize()
                lat.append(e0.elapsed_time(e1) * 1e3)
            nbytes = m * k * 2 + sum(n * k / 2 + n * (k // group) * 2 + (r * k + n * r) * 2
                                     + m * n * 2 for n in ns)
            out.append({"group": name, "m": m, "k": k, "n": list(ns),
                        "us_per_call": round(us_multi, 2), "separate_us": round(us_sep, 2),
                        "p50_us": round(float(np.median(lat)), 2),
                        "gbs": round(nbytes / (us_multi * 1e-6) / 1e9, 1),
                        "frac_hbm": round(nbytes / (us_multi * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del pool, base
        torch.cuda.empty_cache()
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path would shard tokens across GPUs with one dA/dB all-reduce per linear)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    from representax_amd import _native

    _native.load()
    dev = torch.device("cuda:0")
    use_graph = not args.no_graph

    if args.only == "int4lora":
        print(json.dumps(run_int4lora(args.steps, args.warmup, use_graph)))
        return
    if args.only == "skinny":
        print(json.dumps(run_skinny()))
        return
    if args.only == "bert":
        line = run_bert()
        line["roofline"] = step_linear_roofline(bert_linear_rooflines(), "full")
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = trainstep_cpu_baseline(BERT_STEP_LINEARS, 12, 16, 64, 512)
        print(json.dumps(line))
        return
    if args.only == "qwen3":
        line = run_qwen3()
        line["roofline"] = step_linear_roofline(qwen3_linear_rooflines(), "full")
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = trainstep_cpu_baseline(QWEN3_STEP_LINEARS, 28, 32, 64, 128)
        print(json.dumps(line))
        return
    if args.only == "copyref":
        run_copyref()
        return
    if args.only == "int4shapes":
        run_int4_shapes()
        return
    if args.only == "castref":
        run_castref(fp8_setup(args.tokens, dev))
        return
    if args.only == "vendor":
        run_vendor(fp8_setup(args.tokens, dev))
        return
    if args.only == "fp8gemm":
        run_fp8gemm_only(fp8_setup(args.tokens, dev))
        return
    if args.only == "fp8delayed":
        print(json.dumps(run_fp8_delayed(fp8_setup(args.tokens, dev), args.tokens, args.steps,
                                         args.warmup, use_graph)))
        return

    log("fp8: setting up inputs")
    layers = fp8_setup(args.tokens, dev)
    fn, mode = maybe_graph(fp8_step_fn(layers), use_graph)
    log(f"fp8: timing {args.steps} steps ({mode})")
    ms = time_region(fn, args.steps, args.warmup)
    value = fp8_flops(args.tokens) / (ms * 1e-3) / 1e12
    log(f"fp8: {ms:.3f} ms/step, {value:.1f} TFLOP/s; timing GEMM launches")
    roofline = fp8_gemm_roofline(layers)
    quantize = fp8_quantize_report(layers, ms, roofline["gemm_us_per_step"])
    result = {
        "metric": "INT4-LoRA/FP8 linear TFLOP/s & % roofline; train-step tokens/sec, 1 GPU",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3/e5m2 (f32 accumulate, bf16 out)",
        "data": "synthetic",
        "config": {
            "workload": "fp8 e4m3 linear fwd+bwd, dynamic per-tensor amax, BERT-base shapes "
                        "768->768 x4, 768->3072, 3072->768",
            "tokens": args.tokens,
            "x": "bf16 ~N(0,1), 0.1% outliers x50",
            "w": "bf16 ~N(0,0.02)",
            "mode": mode,
        },
        "roofline": roofline,
        "quantize": quantize,
    }
    if args.only is None and not args.no_secondary:
        log("fp8 with delayed scaling")
        delayed = run_fp8_delayed(layers, args.tokens, args.steps, args.warmup, use_graph)
        del layers, fn
        torch.cuda.empty_cache()
        log("int4lora: per-row and group-64")
        i4_row = run_int4lora(args.steps, args.warmup, use_graph)
        i4_grp = run_int4lora(args.steps, args.warmup, use_graph, group_size=64)
        result["secondary"] = [delayed, i4_row, i4_grp]
        log("skinny-M sweep")
        skinny = run_skinny()
        result["secondary"].append(skinny)
        log("bert-base int4-lora train step (full remat), per-linear rooflines, no-remat step")
        bert = run_bert()
        bert["roofline"] = step_linear_roofline(bert_linear_rooflines(), "full")
        result["secondary"] += [bert, run_bert(remat="none")]
        log("qwen3-shaped int4-lora train step (full remat), per-linear rooflines, no-remat step")
        qwen3 = run_qwen3()
        qwen3["roofline"] = step_linear_roofline(qwen3_linear_rooflines(), "full")
        result["secondary"] += [qwen3, run_qwen3(remat="none")]
        if not args.no_cpu_baseline:
            log("cpu baselines of the int4-lora, skinny and train-step lines (numpy oracle)")
            i4_row["cpu_baseline"] = int4lora_cpu_baseline()
            skinny["cpu_baseline"] = skinny_cpu_baseline()
            bert["cpu_baseline"] = trainstep_cpu_baseline(BERT_STEP_LINEARS, 12, 16, 64, 512)
            qwen3["cpu_baseline"] = trainstep_cpu_baseline(QWEN3_STEP_LINEARS, 28, 32, 64, 128)
    if args.only is None and not args.no_cpu_baseline:
        log("cpu baseline (numpy oracle)")
        result["cpu_baseline"] = fp8_cpu_baseline()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
