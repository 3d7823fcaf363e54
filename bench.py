"""Benchmark of the MI355X Qwen3-MoE FFN block (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 30b_t32] [--extra 30b_t1,...]
                    [--graph | --eager]

A step is one MoE block forward (router, top-k, dispatch, experts, combine)
over one batch of T tokens of synthetic input, with weights and inputs
already resident in HBM.  Weights are cycled over L independently generated
layers (and inputs over L token batches) so that no step finds its experts
in the 256 MB MALL or the L2 left warm by the previous steps.  The K timed
steps of a batched workload (T > 1) are one replay of a HIP graph that
captured K library calls (the way a serving loop replays a captured
forward: no host launch cost between the block's kernels), bracketed by
device synchronisations; the eager loop (K library calls from a Python
loop, the way TIE's host loop calls the block) is timed as well and
reported as ms_per_step_eager.  One-token workloads are timed eagerly: under
capture they take their three-launch form, and the one-launch kernel is
what the host loop runs.  --eager times every workload eagerly, --graph
every workload as a graph replay.

Prints one JSON line: the headline workload (`value`, tokens/s), the
roofline of its dominant kernel (event-timed on the library's stream), the
CPU baseline (TIE's own compiled MoE path on the host cores, or the C
restatement when the reference build cannot run here) with the parity of
the GPU's outputs against it on the same tokens, and the same for the
extra workloads named by --extra.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
FP32_VALU_TFLOPS = 157.3    # MI355X fp32 (packed) vector peak


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- workloads
def gen_device_layer(torch, cfg, seed):
    """GGUF-layout tensors for one layer, generated on the GPU (same
    distributions as tie_amd.synth, different random stream)."""
    from tie_amd import synth
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    d, F, E = cfg["d"], cfg["F"], cfg["E"]
    dev = "cuda"

    def half_abs(n):
        return (torch.randn(n, generator=g, device=dev) * 0.01).abs().half().view(torch.uint8).reshape(n, 2)

    def expert(wtype, rows, inn):
        if wtype == synth.BF16:
            w = torch.randn(E * rows * inn, generator=g, device=dev) * 0.02
            return w.to(torch.bfloat16).view(torch.uint8)
        nb = E * rows * (inn // 256)
        if wtype == synth.Q4_K:
            b = torch.randint(0, 256, (nb, 144), generator=g, device=dev, dtype=torch.uint8)
            b[:, 0:2] = half_abs(nb)
            b[:, 2:4] = half_abs(nb)
        else:
            b = torch.randint(0, 256, (nb, 210), generator=g, device=dev, dtype=torch.uint8)
            b[:, 192:208] = torch.randint(-32, 32, (nb, 16), generator=g, device=dev,
                                          dtype=torch.int8).view(torch.uint8)
            b[:, 208:210] = half_abs(nb)
        return b.reshape(-1)

    router = torch.randn(E, d, generator=g, device=dev) * 0.02
    gate = expert(cfg["gu_type"], F, d)
    up = expert(cfg["gu_type"], F, d)
    down = expert(cfg["down_type"], d, F)
    bias = pbias = None
    if cfg.get("zipf"):
        bias = torch.from_numpy(synth.zipf_bias(E, s=cfg["zipf"], seed=seed + 7)).to(dev)
    if cfg.get("probs_bias"):
        pbias = torch.randn(E, generator=g, device=dev) * cfg["probs_bias"]
    return router, gate, up, down, bias, pbias


class Workload:
    def __init__(self, torch, tie_amd, cfg, n_layers, seed0=4242):
        from tie_amd import synth
        self.cfg = cfg
        self.layers = []
        self.layer_bytes = 0
        self.host_layer0 = None  # layer 0's GGUF-layout tensors on the host (the CPU leg's weights)
        for i in range(n_layers):
            r, g, u, dn, b, pb = gen_device_layer(torch, cfg, seed0 + 17 * i)
            L = tie_amd.Layer(cfg["d"], cfg["F"], cfg["E"], r, g, u, dn, cfg["gu_type"], cfg["gu_type"],
                              cfg["down_type"], bias=b, on_device=True, routing=cfg.get("routing", 0),
                              probs_bias=pb)
            if i == 0:
                host = lambda t: None if t is None else t.cpu().numpy()  # noqa: E731
                self.host_layer0 = synth.MoELayer(cfg["d"], cfg["F"], cfg["E"], host(g), host(u), host(dn),
                                                  host(r), cfg["gu_type"], cfg["down_type"], host(b),
                                                  cfg.get("routing", 0), host(pb))
            self.layer_bytes = L.nbytes()
            self.layers.append(L)
            del r, g, u, dn
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def run_dense(torch, tie_amd, cfg, steps, warmup, n_copies, flags):
    """dispatch_mat_mat through tie_hip_mat_mat: T rows of x times one
    [rows][in] weight matrix, cycling `n_copies` matrices so the MALL does
    not hold the weights.  Same result fields as run_config."""
    from tie_amd import synth
    rows, in_dim, T, wtype = cfg["rows"], cfg["in"], cfg["T"], cfg["wtype"]
    g = torch.Generator(device="cuda")
    g.manual_seed(cfg["seed"])
    mats = []
    for i in range(n_copies):
        if wtype == synth.F32:
            w = torch.randn(rows * in_dim, generator=g, device="cuda") * 0.02
        else:
            rng = np.random.default_rng(cfg["seed"] + i)
            w = torch.from_numpy(synth.expert_tensor(rng, wtype, 1, rows, in_dim)).cuda()
        mats.append(tie_amd.Matrix(w, wtype, rows, in_dim, on_device=True))
        del w
    X = torch.randn(n_copies, T, in_dim, generator=g, device="cuda")
    out = torch.empty(T, rows, device="cuda")

    # the calls go on torch's current stream, so that two events on it
    # bracket the timed calls (one call is one kernel, or three on the
    # matrix cores: its average duration is the events' interval / steps;
    # events around every call would add their own gaps)
    cs = torch.cuda.Stream()  # a stream of its own (handle 0 would mean the library's stream)

    def step(s):
        mats[s % n_copies].mat_mat(X[s % n_copies], T, out, flags=flags, stream=cs.cuda_stream)

    for s in range(warmup):
        step(s)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(cs)
    for s in range(steps):
        step(s)
    e1.record(cs)
    torch.cuda.synchronize()
    ms = 1e3 * (time.perf_counter() - t0) / steps
    # which path ran (the library's per-call profile names it)
    tie_amd.profile_enable(True)
    step(0)
    prof = tie_amd.profile_read()
    tie_amd.profile_enable(False)
    wbytes = rows * synth.row_bytes(wtype, in_dim)
    nbytes = wbytes + T * in_dim * 4 + T * rows * 4
    flops = 2.0 * T * rows * in_dim
    key = "dense_mfma" if "dense_mfma" in prof else "dense"
    n = steps
    avg_ms = e0.elapsed_time(e1) / steps
    kernels = {key: {"avg_us": round(1e3 * avg_ms, 3), "launches": n, "alg_bytes": nbytes,
                         "GBps": round(nbytes / (avg_ms * 1e-3) / 1e9, 1), "alg_flops": flops,
                         "TFLOPs": round(flops / (avg_ms * 1e-3) / 1e12, 2)}}
    for mt in mats:
        mt.close()
    return dict(T=T, k=0, ms=ms, tokens_per_s=T / (ms * 1e-3), U=1, block_bytes=nbytes, block_flops=flops,
                block_GBps=nbytes / (ms * 1e-3) / 1e9, block_TFLOPs=flops / (ms * 1e-3) / 1e12, kernels=kernels,
                layers=n_copies, ms_eager=ms, timing="eager")


def expert_bytes(cfg):
    """HBM bytes of one expert: gate + up together, and down."""
    from tie_amd import synth
    gu = 2 * cfg["F"] * synth.row_bytes(cfg["gu_type"], cfg["d"])
    dn = cfg["d"] * synth.row_bytes(cfg["down_type"], cfg["F"])
    return gu, dn


def run_config(torch, tie_amd, wl, T, k, steps, warmup, flags, cfg=None, graph=False):
    """Times `steps` forwards of T tokens; returns the measurement dict.
    cfg: the workload config (default: the one the layers were made for).
    graph: also time the steps as one replay of a captured HIP graph and
    report that (the eager loop's time is reported either way)."""
    from tie_amd import synth
    cfg = cfg or wl.cfg
    d, F, E = cfg["d"], cfg["F"], cfg["E"]
    nL = len(wl.layers)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    X = torch.randn(nL, T, d, generator=gen, device="cuda")
    out = torch.empty(T, d, device="cuda")
    idx = torch.empty(nL, T, k, dtype=torch.int32, device="cuda")
    w = torch.empty(nL, T, k, device="cuda")

    residual = bool(cfg.get("residual"))
    if residual:
        # the FFN half of the layer: out = X[l] + block(rms_norm(X[l])) (out
        # of place, so every step sees the same inputs)
        norm = torch.from_numpy(synth.make_norm_weight(cfg["seed"], d)).cuda()

    def step(s, record_topk=False, stream=None):
        l = s % nL
        if residual:
            wl.layers[l].forward_residual(X[l], norm, 1e-6, T, k, out, idx[l] if record_topk else None,
                                          w[l] if record_topk else None, flags=flags, stream=stream)
            return
        wl.layers[l].forward(X[l], T, k, out, idx[l] if record_topk else None, w[l] if record_topk else None,
                             flags=flags, stream=stream)

    for s in range(nL):  # routing of every (layer, batch) pair, for the byte counts
        step(s, record_topk=True)
    torch.cuda.synchronize()
    # layer 0 on batch 0: the outputs the parity check compares with TIE's
    # CPU path (step 0 wrote them last for layer 0 only when nL == 1)
    step(0, record_topk=True)
    torch.cuda.synchronize()
    gpu_out0 = (X[0].cpu().numpy(), out.cpu().numpy(), idx[0].cpu().numpy(), w[0].cpu().numpy())
    # eager: one library call per step from this Python loop (host launch
    # overhead included), on a stream of our own with two events inside the
    # host clock's bracket (the GPU interval of the same steps)
    es = torch.cuda.Stream()
    for s in range(warmup):
        step(s, stream=es.cuda_stream)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(es)
    for s in range(steps):
        step(s, stream=es.cuda_stream)
    ev1.record(es)
    torch.cuda.synchronize()
    ms_eager = 1e3 * (time.perf_counter() - t0) / steps
    gpu_ms_eager = ev0.elapsed_time(ev1)
    ms = ms_eager
    timing = "eager"
    if graph:
        # the same `steps` forwards captured once as a HIP graph on a stream
        # of their own (its workspace sized by the warm-up) and replayed: the
        # GPU's time per step without the host's launch cost.  A capture
        # that fails leaves the eager time as the result (and says why).
        try:
            gs = torch.cuda.Stream()
            with torch.cuda.stream(gs):
                for s in range(max(warmup, nL)):
                    step(s, stream=gs.cuda_stream)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=gs, capture_error_mode="thread_local"):
                for s in range(steps):
                    step(s, stream=gs.cuda_stream)
            g.replay()  # warm-up replay
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            g.replay()
            torch.cuda.synchronize()
            ms = 1e3 * (time.perf_counter() - t0) / steps
            timing = "graph"
            del g
        except Exception as exc:  # noqa: BLE001 -- any capture failure falls back to the eager time
            torch.cuda.synchronize()
            log("graph capture failed (%s): reporting the eager time" % exc)
            timing = "eager (graph capture failed: %s)" % type(exc).__name__

    # per-kernel timing over the same sequence of steps, from events bound to
    # each kernel's own dispatch; the device is drained after every step so
    # that no dispatch waits in the queue behind the previous step's kernels
    # (a one-token step is one kernel, and its start event would otherwise
    # include that wait)
    tie_amd.profile_enable(True)
    for s in range(steps):
        step(s)
        torch.cuda.synchronize()
    prof = tie_amd.profile_read()
    tie_amd.profile_enable(False)
    if len(prof) == 1 and next(iter(prof.values()))[1] == steps and timing == "eager":
        # a step of one kernel (the one-token block): its steady-state
        # duration is the per-launch time of the timed loop's back-to-back
        # launches, from the events inside its host-clock bracket (a
        # dispatch-bound event pair also counts the end-of-kernel release,
        # which back-to-back launches overlap with the next start)
        prof = {next(iter(prof)): (gpu_ms_eager, steps)}
    tie_amd.stream_release(es.cuda_stream)

    idx_h = idx.cpu().numpy()
    U = np.array([len(np.unique(idx_h[l][idx_h[l] >= 0])) for l in range(nL)], np.float64)
    U_avg = float(np.mean([U[s % nL] for s in range(steps)]))
    gu_b, dn_b = expert_bytes(cfg)
    pairs = T * k
    y_bytes = 4  # the MFMA path's y: fp32
    h_bytes = 2 if cfg["down_type"] != synth.BF16 else 4  # h: f16 (quantised down) or bf16 hi + lo
    kern_bytes = {
        "router": E * d * 4 + T * d * 4,
        "exact_gate_up": U_avg * gu_b + T * d * 4 + pairs * F * 4,
        "exact_down": U_avg * dn_b + pairs * F * 4 + pairs * d * 4,
        "decode_gate_up": U_avg * gu_b + T * d * 4 + pairs * F * 4,
        "decode_down": U_avg * dn_b + pairs * F * 4 + T * d * 4 * (2 if residual else 1),
        "decode_one": E * d * 4 + U_avg * (gu_b + dn_b) + T * d * 4 * (3 if residual else 2),
        "combine": pairs * d * 4 + T * d * 4 * (3 if residual else 1),
        "rmsnorm": 2 * T * d * 4 + d * 4,
        "dispatch": pairs * 4 * 2,
        "mfma_gate_up": U_avg * gu_b + T * d * 2 + pairs * F * h_bytes,
        "mfma_down": U_avg * dn_b + pairs * F * h_bytes + pairs * d * y_bytes,
    }
    kern_flops = {
        "mfma_gate_up": 2.0 * pairs * 2 * F * d,
        "mfma_down": 2.0 * pairs * F * d,
        "exact_gate_up": 2.0 * pairs * 2 * F * d,
        "exact_down": 2.0 * pairs * F * d,
        "decode_gate_up": 2.0 * pairs * 2 * F * d,
        "decode_down": 2.0 * pairs * F * d,
        "decode_one": 2.0 * T * (E * d + 3 * k * F * d),
        "router": 2.0 * T * E * d,
    }
    block_bytes = E * d * 4 + U_avg * (gu_b + dn_b) + 2 * T * d * 4
    block_flops = T * (2 * E * d + k * 6 * d * F)
    kernels = {}
    for name, (tot, n) in prof.items():
        if n == 0:
            continue
        avg_ms = tot / n
        kb = kern_bytes.get(name)
        kf = kern_flops.get(name)
        kernels[name] = {"avg_us": round(1e3 * avg_ms, 3), "launches": n,
                         "alg_bytes": kb, "GBps": round(kb / (avg_ms * 1e-3) / 1e9, 1) if kb else None,
                         "alg_flops": kf, "TFLOPs": round(kf / (avg_ms * 1e-3) / 1e12, 2) if kf else None}
    return dict(T=T, k=k, ms=ms, tokens_per_s=T / (ms * 1e-3), U=U_avg, block_bytes=block_bytes,
                block_flops=block_flops, block_GBps=block_bytes / (ms * 1e-3) / 1e9,
                block_TFLOPs=block_flops / (ms * 1e-3) / 1e12, kernels=kernels, layers=nL, gpu_out0=gpu_out0,
                ms_eager=ms_eager, timing=timing)


def workload_name(synth, name, cfg):
    if cfg.get("kind") == "dense":
        return "%s: dense %s %d x %d, T=%d" % (name, synth.TYPE_NAMES[cfg["wtype"]], cfg["rows"], cfg["in"], cfg["T"])
    return "%s: d=%d F=%d E=%d k=%d T=%d, gate/up %s, down %s" % (
        name, cfg["d"], cfg["F"], cfg["E"], cfg["k"], cfg["T"], synth.TYPE_NAMES[cfg["gu_type"]],
        synth.TYPE_NAMES[cfg["down_type"]])


def compute_dtype(m, cfg):
    """Operand type of the workload's expert products: f16 (Q4_K / Q6_K
    weights on the matrix cores, fp32 accumulation), bf16 (BF16 weights on
    the matrix cores, activations split into two bf16 parts), or f32 (TIE's
    exact fp32 arithmetic)."""
    from tie_amd import synth
    if any("mfma" in k for k in m["kernels"]):
        return "bf16" if cfg.get("gu_type", cfg.get("wtype")) == synth.BF16 else "f16"
    return "f32"


def roofline(m, config):
    """Roofline object for the dominant (longest) kernel of a measurement of one
    workload; traffic is the copy-scaled HBM bytes per launch measured for that
    kernel on that workload (None when not profiled)."""
    # (kernels without an algorithmic byte count -- the exact recomputation
    # of out-of-range tokens, which runs empty on these inputs -- are not
    # candidates)
    name, kd = max(((n, v) for n, v in m["kernels"].items() if v.get("alg_bytes")), key=lambda kv: kv[1]["avg_us"])
    traffic = None
    # the dominant kernel's event-timed duration must fit in a step
    kernel_le_step = kd["avg_us"] <= 1e3 * m["ms"]
    tfile = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            t = json.load(f)
        traffic = t.get("%s@%s" % (name, config))
    # bound: MFMA when the kernel runs on the matrix cores and its algorithmic
    # intensity is above the MI355X ridge point (2.5 PFLOP/s / 8 TB/s)
    ridge = BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    mfma = "mfma" in name and kd.get("alg_flops") and kd["alg_flops"] / kd["alg_bytes"] > ridge
    if mfma:
        return {"kernel": name, "bound": "mfma", "achieved": kd["TFLOPs"], "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(kd["TFLOPs"] / BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                "alg_flops_per_launch": kd["alg_flops"], "alg_bytes_per_launch": kd["alg_bytes"],
                "avg_us": kd["avg_us"], "kernel_le_step": kernel_le_step}
    achieved = kd["GBps"]
    return {"kernel": name, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "alg_bytes_per_launch": kd["alg_bytes"], "avg_us": kd["avg_us"], "kernel_le_step": kernel_le_step}


# ---------------------------------------------------------------- CPU baseline
def cpu_has(flag):
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return flag in line.split()
    except OSError:
        pass
    return False


def cpu_pool_threads():
    """TIE's thread-pool size for the CPU leg: min(nproc, 32), at least k = 8
    (model_qwen3.c:413 indexes tasks[num_threads] by slot), and no more than
    this process's CPU share (OMP_NUM_THREADS, which the GPU box sets to it)."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count() or 8
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or nproc
    return max(8, min(nproc, share, 32)), nproc


def cpu_baseline(cfg, layer, x_gpu, gpu, budget_s):
    """TIE's MoE path on the host cores (the reference's own sources compiled,
    oracle/_ref, kind "reference", when its build runs on this CPU; else the
    C restatement, kind "port") on layer 0 of the GPU workload and a sample
    of the GPU's batch-0 tokens: tokens/s over ~budget_s, and the parity of
    the GPU's outputs for those tokens (from the same forward over the full
    batch) against TIE's:
      routing_mismatch  tokens whose selected experts differ, outside near ties
      near_ties         tokens whose 8th and 9th logits differ by < 1e-5
      max_abs, rel_l2   over the sampled output rows."""
    from oracle import bind
    from tie_amd import synth
    k = cfg["k"]
    T = cfg["T"]
    S = min(T, 32 if cfg["d"] <= 2048 else 16)
    # evenly spaced sample of the batch (the MFMA path groups all T tokens)
    rows = np.unique(np.linspace(0, T - 1, S).round().astype(int))
    xs = np.ascontiguousarray(x_gpu[rows])
    threads, nproc = cpu_pool_threads()
    use_ref = bind.ref_available() and cpu_has("avx512f") and cpu_has("avx2")
    fn = (lambda: bind.ref_moe_block(layer, xs, k, nthreads=threads, with_logits=True)) if use_ref else \
        (lambda: bind.moe_block(layer, xs, k, nthreads=threads, with_logits=True))
    # the reference prints progress on stdout (math_dispatch.c:657): send
    # the C-level stdout to stderr meanwhile, so that stdout carries only the
    # result line
    sys.stdout.flush()
    saved = os.dup(1)
    os.dup2(2, 1)
    try:
        ro, ri, rw, lg = fn()  # warm-up (also builds the reference's thread pool); its outputs are checked
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
    finally:
        os.dup2(saved, 1)
        os.close(saved)
    g_out, g_idx, g_w = gpu
    g_out, g_idx = g_out[rows], g_idx[rows]
    srt = -np.sort(-lg, axis=1)
    near = np.abs(srt[:, k - 1] - srt[:, k]) < 1e-5 if lg.shape[1] > k else np.zeros(len(rows), bool)
    differ = (g_idx != ri).any(axis=1)
    err = np.abs(g_out.astype(np.float64) - ro)
    parity = {"tokens": int(len(rows)), "routing_mismatch": int((differ & ~near).sum()),
              "near_ties": int(near.sum()), "near_tie_mismatch": int((differ & near).sum()),
              "max_abs": float(err.max()), "max_ref": float(np.abs(ro).max()),
              "max_abs_over_max_ref": float(err.max() / max(float(np.abs(ro).max()), 1e-30)),
              "rel_l2": float(np.linalg.norm(err) / max(np.linalg.norm(ro), 1e-30)),
              "against": "reference" if use_ref else "port"}
    base = {"value": round(n * len(rows) / el, 2), "unit": "tokens/s", "cores": threads,
            "kind": "reference" if use_ref else "port",
            "sample": "%d calls of %d tokens (rows of the GPU batch; %s weights, layer 0 of the GPU workload) in "
                      "%.1f s on a %d-thread pool; nproc=%d" % (n, len(rows), synth.TYPE_NAMES[cfg["gu_type"]],
                                                               el, threads, nproc)}
    return base, parity


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="30b_t32")
    ap.add_argument("--extra", default="30b_t1,30b_t2048,30b_bf16_zipf_t512,235b_t1,235b_t1024")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU-leg timing budget of the headline workload (the others get half)")
    ap.add_argument("--layers", type=int, default=0, help="weight layers cycled (0 = auto)")
    ap.add_argument("--path", default="auto", choices=["auto", "exact", "mfma"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time every workload as one replay of a HIP graph that captured the K steps (the default "
                         "for T > 1); under capture one-token forwards take their three-launch form")
    ap.add_argument("--eager", action="store_true",
                    help="time every workload as the eager loop (one library call per step)")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="only run a plain device copy of this many MiB 5 times (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (collectives are out of scope); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_mb:
        n = args.copy_mb << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n, "launches": 5}), flush=True)
        return
    import tie_amd
    from tie_amd import synth
    tie_amd.init(0)
    flags = {"auto": tie_amd.PATH_AUTO, "exact": tie_amd.PATH_EXACT, "mfma": tie_amd.PATH_MFMA}[args.path]

    names = [args.config] + [c for c in args.extra.split(",") if c and c not in (args.config, "none")]
    workloads = {}
    results = {}
    gpu_outs = {}
    for name in names:
        cfg = dict(synth.CONFIGS[name])
        if cfg.get("kind") == "dense":
            steps = max(10, args.steps // 4)
            wbytes = cfg["rows"] * synth.row_bytes(cfg["wtype"], cfg["in"])
            ncp = max(2, min(64, int(1.2e9 // wbytes)))
            log("timing dense %s: %d x %d, T=%d, %d matrices" % (name, cfg["rows"], cfg["in"], cfg["T"], ncp))
            fl = {"exact": tie_amd.PATH_EXACT, "mfma": tie_amd.PATH_MFMA}.get(cfg.get("path"), flags)
            results[name] = run_dense(torch, tie_amd, cfg, steps, max(2, args.warmup // 4), ncp, fl)
            log(json.dumps({name: results[name]}))
            continue
        key = (cfg["d"], cfg["F"], cfg["E"], cfg["gu_type"], cfg["down_type"], cfg.get("zipf"), cfg.get("routing", 0),
               cfg.get("probs_bias"))
        if key not in workloads:
            per_layer = cfg["E"] * sum(expert_bytes(cfg))
            nL = args.layers or max(8, min(40, int(16e9 // per_layer)))
            log("generating %d layers for %s (%.2f GB each)" % (nL, name, per_layer / 1e9))
            workloads[key] = Workload(torch, tie_amd, cfg, nL)
        steps = args.steps if name == args.config else max(10, args.steps // 4)
        warm = args.warmup if name == args.config else max(2, args.warmup // 4)
        log("timing %s: T=%d, %d warm-up + %d steps" % (name, cfg["T"], warm, steps))
        results[name] = run_config(torch, tie_amd, workloads[key], cfg["T"], cfg["k"], steps, warm, flags, cfg,
                                   graph=args.graph or (not args.eager and cfg["T"] > 1))
        gpu_outs[name] = (key, results[name].pop("gpu_out0"))
        log(json.dumps({name: results[name]}))

    # CPU legs (TIE's path on the host cores, same weights and tokens) and
    # the parity of the GPU outputs against it, per workload
    cpu, parity = {}, {}
    for name in names:
        cfg = synth.CONFIGS[name]
        if args.no_cpu or name not in gpu_outs or cfg.get("residual"):
            cpu[name], parity[name] = None, None
            continue
        key, (x0, out0, idx0, w0) = gpu_outs[name]
        budget = args.cpu_seconds if name == args.config else args.cpu_seconds / 2
        log("cpu baseline %s ..." % name)
        cpu[name], parity[name] = cpu_baseline(cfg, workloads[key].host_layer0, x0, (out0, idx0, w0), budget)
        log(json.dumps({name: {"cpu_baseline": cpu[name], "parity": parity[name]}}))

    main_name = args.config
    m = results[main_name]
    cfg = synth.CONFIGS[main_name]
    extra = {}
    for name in names[1:]:
        r = results[name]
        extra[name] = {"tokens_per_s": round(r["tokens_per_s"], 1), "ms_per_step": round(r["ms"], 4),
                       "dtype": compute_dtype(r, synth.CONFIGS[name]),
                       "ms_per_step_eager": round(r["ms_eager"], 4), "timing": r["timing"],
                       "block_GBps": round(r["block_GBps"], 1), "block_TFLOPs": round(r["block_TFLOPs"], 3),
                       "roofline": roofline(r, name), "cpu_baseline": cpu.get(name), "parity": parity.get(name),
                       "kernels": r["kernels"]}
    line = {
        "metric": "MoE block tokens/s; HBM GB/s at T=1, MFMA TFLOP/s at T=2048 (30B-A3B)",
        "value": round(m["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["ms"], 4),
        "ms_per_step_eager": round(m["ms_eager"], 4),
        "timing": m["timing"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": compute_dtype(m, cfg),
        "data": "synthetic (seeded GGUF-layout Q4_K/Q6_K blocks, N(0,1) inputs; %d weight layers cycled)" % m[
            "layers"],
        "config": {"workload": workload_name(synth, main_name, cfg), "T": cfg["T"], "path": args.path},
        "roofline": roofline(m, main_name),
        "cpu_baseline": cpu.get(main_name),
        "parity": parity.get(main_name),
        "block_GBps": round(m["block_GBps"], 1),
        "distinct_experts_per_step": round(m["U"], 2),
        "kernels": m["kernels"],
        "extra": extra,
    }
    # the two figures BASELINE's metric is quoted on: the 30B block at T=1
    # (HBM GB/s of its algorithmic bytes) and at T=2048 (MFMA TFLOP/s)
    if "30b_t1" in results:
        line["t1_block_GBps"] = round(results["30b_t1"]["block_GBps"], 1)
        line["t1_block_hbm_frac"] = round(results["30b_t1"]["block_GBps"] / HBM_PEAK_GBS, 4)
    if "30b_t2048" in results:
        line["t2048_block_TFLOPs"] = round(results["30b_t2048"]["block_TFLOPs"], 2)
        line["t2048_block_mfma_frac"] = round(results["30b_t2048"]["block_TFLOPs"] / BF16_PEAK_TFLOPS, 4)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
