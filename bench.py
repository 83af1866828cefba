"""MoE-layer throughput on one MI355X.

A step is one ``DeepSeekMoE.forward`` (router GEMM, routing, permutation,
grouped gate/up + SwiGLU GEMM, grouped down GEMM, combine) over one batch of
the workload's synthetic tokens, with inputs and weights resident in HBM.

Prints one JSON line:
  value           tokens/s of the whole layer forward (timed K steps)
  gemm_tflops     algorithmic expert-GEMM FLOPs (6*T*k*D*F) / (gate_up + down
                  kernel time), and its fraction of the 2.5 PFLOP/s dense-bf16
                  matrix-core peak
  roofline        the dominant kernel (grouped gate/up GEMM): algorithmic
                  FLOPs (or bytes) per launch / its average launch time,
                  measured with HIP events on the launch stream around each
                  launch in an instrumented pass of the layer forward; for a
                  launch under 0.2 ms, whose events would add the gaps around
                  it, around back-to-back launches of the same call on the
                  same inputs replayed from one HIP graph instead (longer
                  GEMMs run back to back at a lower clock than in the layer:
                  up to 30 % slower at 0.5 ms)
  kernels_ms      average time of every stage
  cpu_baseline    the reference path (the oracle's torch restatement of
                  mlp.py:64-100) on the host CPU, on a bounded token sample of
                  the same layer, with every host core the process may use
  parity          the timed configuration's output, routing and permutation
                  against the oracle on the same device (outside the timed
                  region): routing and permutation bit-exact flags, the plain
                  allclose pass fraction and the max normalised error; and
                  the layer's output and the oracle's against an fp64 truth
                  of the same inputs (every intermediate unrounded): each
                  one's plain-tolerance failures, max normalised and RMS
                  error (truth_*)
  vs_hipblaslt    (--vs-hipblaslt) the grouped GEMMs' TFLOP/s against
                  torch's F.linear (hipBLASLt) per expert on the same rows
                  and weights, on the workload's routing and a balanced one
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

# Bytes moved between L2 and memory per launch of the dominant kernel (the
# grouped gate/up GEMM), measured with rocprofv3 --pmc: FETCH_SIZE x 2 +
# WRITE_SIZE (KiB, median per dispatch). A device copy in the same run reads
# back as FETCH_SIZE = half and WRITE_SIZE = all of its bytes (FETCH_SIZE
# counts this part's 128-byte read requests as 64 bytes), hence the 2. These
# are constants from the counter passes recorded in profiles/moe_layer_*.md
# (TRAFFIC_SOURCE), not measured by this run: a counter pass needs the
# profiler around the process.
MEASURED_TRAFFIC_BYTES: dict[str, float] = {
    "moe_bf16_d4096_f14336_e8_k2_t16384": (5979173.2 * 2 + 917618.0) * 1024,
    "moe_bf16_d2048_f1408_e64_k6_t8192": (1192495.2 * 2 + 135201.3) * 1024,
    "moe_bf16_d2048_f1408_e64_k6_t8192_zipf": (1069864.4 * 2 + 135200.6) * 1024,
    "moe_bf16_d4096_f1536_e128_k8_t64": (1543036.9 * 2 + 1538.1) * 1024,
    "moe_bf16_d4096_f1536_e128_k8_t1024": (1682144.4 * 2 + 24587.0) * 1024,
    "moe_fp32_d512_f1024_e8_k2_t1024": (73347.5 * 2 + 8195.6) * 1024,
}


TRAFFIC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE passes of bench.py on this workload, "
                  "profiles/moe_layer_<workload>.md (a constant from that profiled run on another MI355X box, "
                  "2026-12-02, scaled by a 1 GiB copy probe; not measured here)")


def _parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default=None, help="workload name (default: the Mixtral-shaped layer)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-parity", action="store_true", help="skip the parity check against the oracle")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU work for the baseline sample")
    p.add_argument("--backward", action="store_true",
                   help="also time forward + backward (reported as train_*; value stays the forward)")
    p.add_argument("--graph", action="store_true",
                   help="also time the step as a replayed HIP graph (reported as graph_*; value stays eager)")
    p.add_argument("--pack", action="store_true",
                   help="read the layer's packed inference copy of the expert weights (opt-in)")
    p.add_argument("--vs-hipblaslt", action="store_true",
                   help="also time the grouped GEMMs against torch's F.linear (hipBLASLt) per expert on the same "
                        "rows and weights, on the workload's routing and on a balanced one (reported as "
                        "vs_hipblaslt)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="before timing, copy a buffer of this many MiB once (a plain copy kernel of known size "
                        "that scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings)")
    return p.parse_args()


class StageTimer:
    """Wraps the ops entry points to record HIP events around each launch on
    the current stream (the stream the kernels are enqueued on)."""

    STAGES = ("moe_route", "moe_permute", "moe_gemm_gate_up", "moe_gemm_gate_up_gather", "moe_gemm_down",
              "moe_combine")
    # the gate/up GEMM reading x through the permutation counts as the gate/up stage
    MERGE = {"moe_gemm_gate_up_gather": "moe_gemm_gate_up"}

    def __init__(self, ops):
        self.ops = ops
        self.orig = {}
        self.events: dict[str, list] = {s: [] for s in self.STAGES}
        self.last_call: dict[str, tuple] = {}

    def __enter__(self):
        for name in self.STAGES:
            fn = getattr(self.ops, name)
            self.orig[name] = fn

            def wrapped(*a, _fn=fn, _name=name, **k):
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                out = _fn(*a, **k)
                e.record()
                self.events[_name].append((s, e))
                self.last_call[self.MERGE.get(_name, _name)] = (_fn, a, k)
                return out

            setattr(self.ops, name, wrapped)
        return self

    def __exit__(self, *exc):
        for name, fn in self.orig.items():
            setattr(self.ops, name, fn)

    def avg_ms(self) -> dict[str, float]:
        events: dict[str, list] = {}
        for k, v in self.events.items():
            events.setdefault(self.MERGE.get(k, k), []).extend(v)
        return {k: (sum(s.elapsed_time(e) for s, e in v) / len(v) if v else 0.0) for k, v in events.items()}


def back_to_back_ms(call, est_ms: float) -> tuple[float, int]:
    """Average duration of one call's kernel over n back-to-back launches of
    the same call on the same inputs, captured in one HIP graph and replayed
    between two HIP events on the replay stream (n sized to about 2 ms of
    work). Returns (ms per launch, n)."""
    fn, a, k = call
    n = max(2, min(50, int(2.0 / max(est_ms, 1e-3))))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn(*a, **k)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(n):
                fn(*a, **k)
        graph.replay()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        times = []
        for _ in range(3):
            s.record(stream)
            graph.replay()
            e.record(stream)
            e.synchronize()
            times.append(s.elapsed_time(e) / n)
    torch.cuda.current_stream().wait_stream(stream)
    del graph
    return sorted(times)[1], n


def host_cores() -> tuple[int, dict]:
    """Threads for the CPU baseline: every CPU in the process's affinity mask,
    capped by the container's CPU quota and by the job's thread budget
    (``OMP_NUM_THREADS``) when either is set — threads beyond the CPUs the job
    is granted only time-slice. Returns (threads, the figures it came from)."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    omp_n = int(omp) if omp and omp.isdigit() and int(omp) > 0 else None
    cores = affinity
    if quota is not None:
        cores = min(cores, max(1, int(quota + 0.5)))
    if omp_n is not None:
        cores = min(cores, omp_n)
    return cores, {"affinity_cpus": affinity, "cgroup_cpu_quota": quota, "omp_num_threads": omp_n}


def parity_leg(layer, x, w, ops) -> dict:
    """Checker leg, outside the timed region: the timed configuration's layer
    output, the route kernel's expert sets and weights and the permutation's
    row order and offsets against the oracle on the same device."""
    from oracle import parity as P

    with torch.inference_mode():
        out = layer(x)
        x_flat = x.view(-1, w.dim)
        route = ops.moe_route(layer.router(x_flat), w.top_k)
        block_m = ops.select_block_m(w.n_tokens, w.n_experts, w.top_k, w.dim, w.dim_ffn, w.dtype)
        perm = ops.moe_permute(route, x_flat, w.n_experts, block_m, copy_rows=False)
        rep = P.layer_parity(layer, x, out, route.topk_idx, route.topk_w, perm.sorted_token, perm.expert_offsets,
                             truth_tokens=0)
    torch.cuda.synchronize()
    return rep


def cpu_baseline(layer, x, w, target_s: float) -> dict:
    """The reference path on the host CPU (bounded token sample)."""
    from oracle import moe_ref as R

    threads, host = host_cores()
    torch.set_num_threads(threads)
    rw, rb, experts, shared = R.module_weights(layer)
    to_cpu = lambda t: None if t is None else t.detach().cpu()  # noqa: E731
    rw, rb = to_cpu(rw), to_cpu(rb)
    experts = [R.ExpertWeights(to_cpu(e.gate), to_cpu(e.up), to_cpu(e.down)) for e in experts]
    x_all = x.view(-1, w.dim)
    n_warm = min(32, x_all.shape[0])
    with torch.no_grad():
        # warm-up, then a calibration sample sized from it, then the timed
        # sample sized to about target_s seconds of CPU work
        n = n_warm
        for _ in range(2):
            xs = x_all[:n].cpu()
            t0 = time.perf_counter()
            R.routed_forward(xs, rw, rb, experts, w.top_k)
            per_tok = max((time.perf_counter() - t0) / n, 1e-7)
            n = int(min(x_all.shape[0], max(n_warm, 0.2 * target_s / per_tok)))
        n = int(min(x_all.shape[0], max(n_warm, target_s / per_tok)))
        # a workload shorter than the target is timed over repeated passes
        reps = max(1, min(2000, round(target_s / (n * per_tok))))
        xs = x_all[:n].cpu()
        t0 = time.perf_counter()
        for _ in range(reps):
            R.routed_forward(xs, rw, rb, experts, w.top_k)
        dt = time.perf_counter() - t0
    passes = f" x {reps} passes" if reps > 1 else ""
    return {
        "value": reps * n / dt,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"first {n} of {x_all.shape[0]} tokens{passes} of the same layer and inputs, reference torch "
                  f"path (mlp.py:79-100) on CPU in {str(w.dtype).replace('torch.', '')}, {dt:.1f} s",
        **host,
    }


def _median_ms(fn, n: int = 12) -> float:
    ts = []
    for _ in range(n):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        e.synchronize()
        ts.append(s.elapsed_time(e))
    ts = ts[2:]
    return sorted(ts)[len(ts) // 2]


def vs_hipblaslt(layer, x, w, ops) -> dict | None:
    """The layer's grouped gate/up (gathering x) and down GEMMs against
    torch's F.linear, i.e. hipBLASLt, run once per expert on the same
    permuted rows and weights (gate and up concatenated into one [2F, D]
    weight, so hipBLASLt's gate/up is one GEMM per expert without the SwiGLU,
    which the grouped kernel fuses): on the workload's routing, and on a
    routing that gives every expert exactly T*k/E rows (token t's j-th slot
    to expert (t*k + j) mod E; whole 256-row tiles when 256 divides it).
    bf16 workloads on 256-row tiles only. Medians of 10 timed calls."""
    import torch.nn.functional as F

    T, E, K, D, Fd = w.n_tokens, w.n_experts, w.top_k, w.dim, w.dim_ffn
    if w.dtype != torch.bfloat16 or ops.select_block_m(T, E, K, D, Fd, w.dtype) != 256:
        return None
    x2 = x.view(-1, D)
    experts = layer.routed_experts
    tg = ops.expert_weight_table([m.gate.weight for m in experts], (Fd, D))
    tu = ops.expert_weight_table([m.up.weight for m in experts], (Fd, D))
    td = ops.expert_weight_table([m.down.weight for m in experts], (D, Fd))
    w_gu = [torch.cat([m.gate.weight, m.up.weight]) for m in experts]
    w_dn = [m.down.weight for m in experts]
    fl_gu, fl_dn = 4.0 * T * K * D * Fd, 2.0 * T * K * D * Fd

    def leg(route) -> dict:
        perm = ops.moe_permute(route, x2, E, 256)
        offs = perm.expert_offsets.tolist()
        h = ops.moe_gemm_gate_up_gather(x2, perm.sorted_token, perm.tiles, tg, tu, E, Fd, 256)
        ours_gu = _median_ms(lambda: ops.moe_gemm_gate_up_gather(x2, perm.sorted_token, perm.tiles, tg, tu, E, Fd, 256))
        ours_dn = _median_ms(lambda: ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, E, D, 256))
        spans = [(e, offs[e], offs[e + 1]) for e in range(E) if offs[e + 1] > offs[e]]
        blas_gu = _median_ms(lambda: [F.linear(perm.x_perm[a:b], w_gu[e]) for e, a, b in spans])
        blas_dn = _median_ms(lambda: [F.linear(h[a:b], w_dn[e]) for e, a, b in spans])
        return {
            "rows_per_expert": [b - a for _, a, b in spans],
            "grouped_gate_up_tflops": fl_gu / ours_gu / 1e9, "grouped_down_tflops": fl_dn / ours_dn / 1e9,
            "hipblaslt_gate_up_tflops": fl_gu / blas_gu / 1e9, "hipblaslt_down_tflops": fl_dn / blas_dn / 1e9,
            "grouped_over_hipblaslt_both": (blas_gu + blas_dn) / (ours_gu + ours_dn),
        }

    with torch.inference_mode():
        real = leg(ops.moe_route(layer.router(x2), K))
        slots = (torch.arange(T, device=x.device).unsqueeze(1) * K + torch.arange(K, device=x.device)) % E
        logits = torch.full((T, E), -8.0, device=x.device)
        logits.scatter_(1, slots, torch.linspace(2.0, 1.0, K, device=x.device).expand(T, K).contiguous())
        balanced = leg(ops.moe_route(logits.to(w.dtype), K))
    torch.cuda.synchronize()
    return {"workload_routing": real, "balanced_routing": balanced,
            "timing": "HIP events around each call (hipBLASLt: one F.linear per expert), median of 10",
            "note": "hipBLASLt's gate/up omits the SwiGLU and its down the routing weight; the grouped kernels fuse both"}


def main():
    args = _parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures the single-GPU MoE layer: every expert is resident on one GPU and the path has no "
            "collectives, so only --gpus 1 is supported.",
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)

    from astrai_amd.extension import ops
    from astrai_amd.workloads import HEADLINE, WORKLOADS, make_layer, routing_stats

    name = args.workload or HEADLINE
    w = WORKLOADS[name]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    layer, x = make_layer(w, dev)
    layer.pack_weights = args.pack
    T = w.n_tokens
    if args.copy_probe_mib:
        src = torch.empty(args.copy_probe_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    with torch.inference_mode():
        for _ in range(args.warmup):
            layer(x)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t_wall = time.perf_counter()
        start.record()
        for _ in range(args.steps):
            out = layer(x)
        end.record()
        torch.cuda.synchronize()
        t_wall = time.perf_counter() - t_wall
        ms_per_step = start.elapsed_time(end) / args.steps

        with StageTimer(ops) as timer:
            for _ in range(args.steps):
                layer(x)
            torch.cuda.synchronize()
        stage_ms = timer.avg_ms()

        logits = layer.router(x.view(-1, w.dim))
        counts = ops.moe_route(logits, w.top_k).chunk_hist.sum(0)
        torch.cuda.synchronize()

        graph_ms = None
        if args.graph:
            graph = torch.cuda.CUDAGraph()
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                layer(x)
                stream.synchronize()
                with torch.cuda.graph(graph, stream=stream):
                    layer(x)
            torch.cuda.current_stream().wait_stream(stream)
            for _ in range(args.warmup):
                graph.replay()
            torch.cuda.synchronize()
            g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            g0.record()
            for _ in range(args.steps):
                graph.replay()
            g1.record()
            torch.cuda.synchronize()
            graph_ms = g0.elapsed_time(g1) / args.steps
    assert torch.isfinite(out.float()).all()

    train_ms = None
    if args.backward:
        layer.requires_grad_(True)
        xg = x.detach().clone().requires_grad_(True)
        dout = torch.randn_like(x)

        params = [p for p in layer.parameters() if p.requires_grad]

        def train_step():
            # gradients cleared from a flat parameter list, as an optimizer's
            # zero_grad(set_to_none=True) does (Module.zero_grad walks the
            # module tree: ~0.8 ms of host time per step at 64 experts)
            for p in params:
                p.grad = None
            xg.grad = None
            layer(xg).backward(dout)

        # the same loop body untimed first (allocator and host caches settle),
        # then at least 10 timed steps: a short loop shows its start-up
        for _ in range(max(2, args.warmup)):
            train_step()
        torch.cuda.synchronize()
        b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n_train = max(10, args.steps)
        b0.record()
        for _ in range(n_train):
            train_step()
        b1.record()
        torch.cuda.synchronize()
        train_ms = b0.elapsed_time(b1) / n_train
        layer.requires_grad_(False)

    bf16 = w.dtype == torch.bfloat16
    gathered = not layer.uses_packed_weights(w.dtype) and ops.gather_supported(T, w.dim, w.dim_ffn, w.dtype)
    s = 2 if bf16 else 4
    peak = PEAK_BF16_TFLOPS if bf16 else PEAK_FP32_TFLOPS
    rows = T * w.top_k
    flops_gate_up = 4.0 * rows * w.dim * w.dim_ffn
    flops_down = 2.0 * rows * w.dim * w.dim_ffn
    t_gu, t_dn = stage_ms["moe_gemm_gate_up"] / 1e3, stage_ms["moe_gemm_down"] / 1e3
    gemm_tflops = (flops_gate_up + flops_down) / (t_gu + t_dn) / 1e12
    t_roof = t_gu  # the dominant kernel's average launch duration
    timing = f"HIP events on the launch stream around each of its {args.steps} launches in the layer forward"
    if t_gu < 2e-4 and "moe_gemm_gate_up" in timer.last_call:
        with torch.inference_mode():
            b2b_ms, n_b2b = back_to_back_ms(timer.last_call["moe_gemm_gate_up"], t_gu * 1e3)
        t_roof = b2b_ms / 1e3
        timing = (f"HIP events on the replay stream around {n_b2b} back-to-back launches of the layer's gate/up "
                  f"call replayed from one HIP graph (median of 3; events around each launch in the layer "
                  f"forward: {t_gu * 1e3:.4f} ms)")
    n_active = int((counts > 0).sum().item())
    weight_bytes = n_active * 3.0 * w.dim * w.dim_ffn * s
    # permutation: the index outputs (routing entries and chunk histograms
    # read; source token, weight and position of every row written) and, when
    # the rows are copied (training, or kernels that cannot gather), x read
    # once and written top_k times. Timed back to back from one HIP graph on
    # the layer's own inputs (a launch of ~10-20 us is shorter than the gaps
    # events add around it), once as the layer runs it and once copying rows.
    n_chunks = -(-T // 32)
    bytes_perm_index = rows * (4 + s) + 4 * w.n_experts * n_chunks + rows * (4 + s + 4)
    bytes_perm_copy = bytes_perm_index + T * w.dim * s + rows * w.dim * s
    perm_call = timer.last_call.get("moe_permute")
    perm_ms = perm_copy_ms = None
    if perm_call is not None:
        fn_p, a_p, k_p = perm_call
        with torch.inference_mode():
            perm_ms, _ = back_to_back_ms(perm_call, max(stage_ms["moe_permute"], 1e-3))
            perm_copy_ms, _ = back_to_back_ms((fn_p, a_p, {**k_p, "copy_rows": True}),
                                              max(stage_ms["moe_permute"], 1e-3))
    bytes_combine = rows * w.dim * s + T * w.dim * s + rows * (s + 8)
    traffic = MEASURED_TRAFFIC_BYTES.get(name)
    block_m = ops.select_block_m(T, w.n_experts, w.top_k, w.dim, w.dim_ffn, w.dtype)
    if bf16 and block_m in (32, 64, 128):
        # decode- and mid-sized loads: the gate/up kernel streams the routed experts' weights
        gu_bytes = n_active * 2.0 * w.dim * w.dim_ffn * s + rows * w.dim * s + rows * w.dim_ffn * s
        gbs = gu_bytes / t_roof / 1e9
        roofline = {"kernel": "gemm_mfma_kernel<gate_up" + (", gather>" if gathered else ">"), "bound": "hbm",
                    "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                    "traffic": traffic, "traffic_source": TRAFFIC_SOURCE if traffic else None,
                    "algorithmic_bytes_per_launch": gu_bytes, "kernel_ms": t_roof * 1e3,
                    "timing": timing}
    else:
        achieved = flops_gate_up / t_roof / 1e12
        if bf16:
            kname = "gemm_stream_kernel<gate_up, gather>" if gathered else "gemm_stream_kernel<gate_up>"
        elif ops.f32_matrix_cores(w.dim, w.dim_ffn, block_m, w.dtype):
            kname = "gemm_f32_mfma_kernel<gate_up>"
        else:
            kname = "gemm_generic_kernel<gate_up>"
        roofline = {"kernel": kname,
                    "bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s", "frac": achieved / peak,
                    "traffic": traffic, "traffic_source": TRAFFIC_SOURCE if traffic else None,
                    "algorithmic_flops_per_launch": flops_gate_up, "kernel_ms": t_roof * 1e3,
                    "timing": timing}

    result = {
        "metric": "MoE-layer tokens/s + grouped-GEMM TFLOP/s (% of bf16 MFMA peak), 1 GPU",
        "value": T / (ms_per_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "wall_s_timed": t_wall,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if bf16 else "f32",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) expert weights, random-init)",
        "config": {**w.describe(), "parallelism": "single GPU, all experts resident",
                   "packed_weights": layer.uses_packed_weights(w.dtype)},
        "gemm_tflops": gemm_tflops,
        "gemm_frac_of_peak": gemm_tflops / peak,
        "roofline": roofline,
        "kernels_ms": stage_ms,
        # with the gathering gate/up GEMM the permutation writes indices only (its rows are read by the GEMM)
        "permute_rows": "gathered by the gate/up GEMM (no x_perm copy)" if gathered else "copied to x_perm",
        "permute": None if perm_ms is None else {
            "as_run_us": perm_ms * 1e3,
            "as_run_gbs": (bytes_perm_copy if not gathered else bytes_perm_index) / (perm_ms / 1e3) / 1e9,
            "copy_rows_us": perm_copy_ms * 1e3,
            "copy_rows_gbs": bytes_perm_copy / (perm_copy_ms / 1e3) / 1e9,
            "algorithmic_bytes": {"index_only": bytes_perm_index, "copy_rows": bytes_perm_copy},
            "peak_gbs": PEAK_HBM_GBS,
            "timing": "back-to-back launches of the layer's permute call (and the same call copying x_perm) "
                      "replayed from one HIP graph, median of 3",
        },
        "combine_gbs": bytes_combine / (stage_ms["moe_combine"] / 1e3) / 1e9,
        "expert_weight_stream_gbs": weight_bytes / (t_gu + t_dn) / 1e9,
        "routing": routing_stats(counts),
    }
    if train_ms is not None:
        result["train_ms_per_step"] = train_ms
        result["train_value"] = T / (train_ms / 1e3)
    if graph_ms is not None:
        result["graph_ms_per_step"] = graph_ms
        result["graph_value"] = T / (graph_ms / 1e3)
    if args.vs_hipblaslt:
        result["vs_hipblaslt"] = vs_hipblaslt(layer, x, w, ops)
    if not args.no_parity:
        result["parity"] = parity_leg(layer, x, w, ops)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(layer, x, w, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
