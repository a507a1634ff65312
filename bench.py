#!/usr/bin/env python3
"""Benchmark of the LTHC interface forward on one MI355X.

One step is one pass of the interface over one synthetic batch at the metric
shape (B=256, 64x64 high-res grid, 16x16 workspace, C=768, L=12, bf16
activations, fp32 weights), with every input resident in HBM before timing:

    Z_0 = R(X_0)                              jit_thc::local_write_traceable
    gamma_l = sum_k alpha * beta_l  (all l)    jit_thc::lazy_gamma_stack
    Z_{l+1} = Z_l + gamma_l * dZ_l  (l < 12)   jit_thc::lazy_workspace_update
    X_L = X_0 + sum_l P_l(dZ_l)                jit_thc::final_accumulate_b4_12_traceable

The dZ_l stand in for the transformer branch outputs (out of scope), so they
are inputs.  `value` is algorithmic bytes per step / time per step, with the
per-op compulsory byte count e*(3T + (4L+1)W) + weights (each op reads each
input once and writes each output once; e = 2, T = B*64*64*C, W = B*256*C).

Prints one JSON line.  `roofline` covers the dominant kernel (the
materialisation), timed with HIP events around each of its launches on the
stream it runs on; `cpu_baseline` times the reference's eager PyTorch op
sequence for the same step (oracle/torch_cpu.py, fp32 CPU tensors) at the
metric shape on the host cores this process may use.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "read/write/materialise HBM GB/s (% of 8 TB/s) at B=256 C=768 bf16; fwd img/s"
PEAK_HBM = 8.0e12
PMC_PROFILE = os.path.join(ROOT, "profiles", "materialise_fwd_b256_pmc.txt")
KERNEL_SOURCES = os.path.join(ROOT, "flowmatching_lthc_amd", "csrc")
KERNEL_HEADER = os.path.join(ROOT, "include", "lthc.h")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--batch", type=int, default=256)
    p.add_argument("--channels", type=int, default=768)
    p.add_argument("--depth", type=int, default=12)
    p.add_argument("--grid", type=int, default=16, help="workspace grid side (high-res side = 4x)")
    p.add_argument("--mode", choices=["graph", "eager"], default="graph", help="how `value` is timed")
    p.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU baseline's metric-shape sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--model-batch", type=int, default=64, help="batch of the LTHC-B/4 forward leg (fwd img/s)")
    p.add_argument("--model-steps", type=int, default=10)
    p.add_argument(
        "--model-name",
        default="lthc_b4_velocity",
        help="build_model name of the model forward leg (the headline figure is lthc_b4_velocity; other names, e.g. "
        "the TriangularLazy or v2 models, for --profile model)",
    )
    p.add_argument("--no-model", action="store_true", help="skip the LTHC-B/4 forward leg")
    p.add_argument("--train-batch", type=int, default=64, help="batch of the interface fwd+bwd leg (configuration 3)")
    p.add_argument("--no-train", action="store_true", help="skip the interface fwd+bwd leg")
    p.add_argument("--no-configs", action="store_true", help="skip the benchmark configuration 2 and 5 legs")
    p.add_argument(
        "--profile",
        choices=[
            "materialise", "read", "recur", "read_multi", "weight_grad", "copy", "model", "train", "triangular",
            "interface_c", "mat_bwd", "interface_bwd", "interface_fwd",
        ],  # fmt: skip
        help="run only this kernel --steps times at the configured shape (for rocprofv3), plus one plain copy "
        "of X0 (a copy kernel of known size that calibrates the FETCH_SIZE / WRITE_SIZE counters); 'model' runs "
        "only the LTHC-B/4 forward leg (without the eager-interface comparison), 'train' only the interface fwd+bwd leg, 'triangular' only the non-shared "
        "interface forward leg, 'interface_c' only the whole-interface C calls at the training batch; 'mat_bwd' is "
        "lthc_materialise_bwd, 'interface_bwd' lthc_interface_bwd (every workspace gradient given) and "
        "'interface_fwd' lthc_interface_fwd (every dZ given) at the configured shape",
    )
    return p.parse_args()


def algorithmic_bytes(B, G, C, L, e=2):
    T = B * (4 * G) ** 2 * C
    W = B * G * G * C
    read = e * (T + W) + 4 * 16 * C
    recur = e * 3 * L * W + 4 * L * C  # + gamma vector per step
    gamma = 4 * 16 * C * (L + 1) + 4 * L * C
    mat = e * (2 * T + L * W) + 4 * 16 * C * L
    return {"read": read, "gamma": gamma, "recur": recur, "materialise": mat, "total": read + gamma + recur + mat}


def kernel_source_sha1():
    """sha1 over every source the library is compiled from: lthc_kernels.hip, the .inc files it includes (in name
    order, each preceded by its name) and include/lthc.h.  The PMC summaries record the one they measured."""
    import hashlib

    h = hashlib.sha1()
    names = sorted(n for n in os.listdir(KERNEL_SOURCES) if n.endswith((".hip", ".inc")))
    for path in [os.path.join(KERNEL_SOURCES, n) for n in names] + [KERNEL_HEADER]:
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def pmc_traffic():
    """HBM bytes per materialise launch from the committed rocprofv3 --pmc summary, and where the figure comes
    from.  The figure is None when the summary is missing or was measured on another kernel source than the one
    built now (its recorded kernel_source_sha1 differs): counters are not collected inside this run."""
    rel_path = os.path.relpath(PMC_PROFILE, ROOT)
    if not os.path.exists(PMC_PROFILE):
        return None, f"no committed PMC summary ({rel_path})"
    text = open(PMC_PROFILE).read()
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    h = re.search(r"kernel_source_sha1:\s*([0-9a-f]+)", text)
    if m is None:
        return None, f"{rel_path} holds no traffic figure"
    if h is None or h.group(1) != kernel_source_sha1():
        return None, f"{rel_path} was measured on another kernel source than this build's: not reported"
    return float(m.group(1)), f"committed rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this kernel source ({rel_path}); not measured in this run"


def host_cpu():
    """(model name, logical CPUs of the host, CPUs this process may run on)."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return name, os.cpu_count() or 1, len(os.sched_getaffinity(0))


def cpu_baseline(B, G, C, L, budget_s):
    """The reference's eager PyTorch op sequence (oracle/torch_cpu.py: SharedLocalRead.read local_thc.py:1211-1223,
    lazy_workspace_update :1325-1328, the write_add loop :1368-1372) on CPU tensors in fp32, at configuration 2
    (B=32, one warm-up step) and then at the metric shape, median time per step.  Threads: the CPUs this process
    may use, capped by OMP_NUM_THREADS (the GPU box's share of its host)."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import torch_cpu as TC

    model, ncpu, share = host_cpu()
    env = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(share, env) if env > 0 else share
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)

    def leg(Bs, budget, max_steps, warm):
        gen = torch.Generator().manual_seed(0)
        H = 4 * G
        x0 = torch.randn((Bs, H, H, C), generator=gen)
        alpha = torch.randn((C, 16), generator=gen) * 0.01 + 1.0 / 16.0
        betas = [torch.randn((C, 16), generator=gen) * 0.02 for _ in range(L)]
        dzs = [torch.randn((Bs, G * G, C), generator=gen) * 0.02 for _ in range(L)]
        with torch.no_grad():
            if warm:
                TC.step(x0, alpha, betas, dzs, G)  # warm-up (allocator, thread pool)
            times, t_start = [], time.perf_counter()
            while len(times) < max_steps and (not times or time.perf_counter() - t_start < budget):
                t0 = time.perf_counter()
                TC.step(x0, alpha, betas, dzs, G)
                times.append(time.perf_counter() - t0)
        times.sort()
        dt = times[len(times) // 2]
        nbytes = algorithmic_bytes(Bs, G, C, L)["total"]
        return {
            "B": Bs,
            "ms_per_step": round(dt * 1e3, 1),
            "steps_timed": len(times),
            "GBps": round(nbytes / dt / 1e9, 3),
        }

    try:  # configuration 2 first: its warm-up step also warms the thread pool for the metric shape's steps
        conf2 = leg(32, max(2.0, budget_s / 4), 10, True)
        metric = leg(B, budget_s, 3, False)
    finally:
        torch.set_num_threads(prev)
    return {
        "value": metric["GBps"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"the reference's eager PyTorch op sequence for the interface (read local_thc.py:1211-1223, {L} "
            f"lazy_workspace_update steps :1325-1328, the write_add loop :1368-1372; oracle/torch_cpu.py) on CPU "
            f"tensors in fp32 at the metric shape B={B} ({metric['steps_timed']} timed step(s) after configuration 2's "
            f"warm-up, median {metric['ms_per_step']} ms); value = the metric's bf16 algorithmic bytes / that time; "
            f"torch.set_num_threads({threads}) on a host of {ncpu} logical CPUs ({model}), {share} of them "
            f"available to this process"
        ),
        "ms_per_step": metric["ms_per_step"],
        "host_cpu_model": model,
        "host_logical_cpus": ncpu,
        "threads": threads,
        "configuration2": conf2,
    }


def c_oracle_baseline(G, C, L, budget_s):
    """The C oracle (fp32 in/out, fp64 accumulate, OpenMP) on a configuration-2 slice of the workload: a secondary
    CPU figure beside the reference's op sequence."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O

    if not os.path.exists(O.LIB):
        O.build()
    share = len(os.sched_getaffinity(0))
    env = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(share, env) if env > 0 else share
    O.set_threads(threads)
    Bs = 32  # the batch of benchmark configuration 2
    d = O.make_inputs(Bs, G, C, L, seed=0)
    x0, alpha = d["x0"], d["alpha"]
    betas, dzs = list(d["beta"]), list(d["dz"])

    def step():
        z = O.Cread(x0, alpha, G)
        gam = O.Cgamma(alpha, betas)
        for l in range(L):
            z = O.Crecur(z, dzs[l], gam[l])
        return O.Cwrite(x0, dzs, betas)

    step()  # warm caches and the OpenMP pool
    n, t0 = 0, time.perf_counter()
    while True:
        step()
        n += 1
        if time.perf_counter() - t0 >= budget_s or n >= 1000:
            break
    dt = (time.perf_counter() - t0) / n
    nbytes = algorithmic_bytes(Bs, G, C, L)["total"]
    return {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "threads": threads,
        "sample": (
            f"C oracle (oracle/lthc_oracle.c, fp32 in/out, fp64 accumulate, OpenMP {threads} threads) running the same "
            f"step (read, gamma, {L} recurrence steps, materialise) on a B={Bs} slice of the workload; {n} steps in "
            f"{dt * n:.1f} s; value = the bf16 algorithmic bytes of that slice / time per step"
        ),
        "ms_per_step": round(dt * 1e3, 3),
    }


def eager_interface(model, torch):
    """The reference's PyTorch op sequence for the interface hooks (local_thc.py:1211-1223 read as a broadcast
    multiply + sum, local_thc.py:1325-1328 recurrence, local_thc.py:1368-1372 materialise as a write_add loop)."""
    g, c = model.workspace_grid, model.hidden_size

    def read(x):
        a = model.shared_read.alpha(dtype=x.dtype)
        cells = x.reshape(x.shape[0], g, 4, g, 4, c).permute(0, 1, 3, 2, 4, 5).reshape(x.shape[0], g * g, 16, c)
        return (cells * a.t()[None, None]).sum(2)

    def write(dz, w):
        cells = dz[:, :, None, :] * w.t()[None, None]
        return cells.reshape(dz.shape[0], g, g, 4, 4, c).permute(0, 1, 3, 2, 4, 5).reshape(dz.shape[0], 4 * g, 4 * g, c)

    model.shared_read.read = read
    model.shared_read.read_with_residual = lambda x: (x, read(x))
    for blk in model.blocks:
        blk.lazy_workspace_update = lambda z, dz, sr, b=blk: z + b.write.gamma_from_alpha(sr.alpha(dtype=dz.dtype))[None, None, :] * dz
        blk.lazy_workspace_step = lambda z, dz, sr, b=blk: (b.lazy_workspace_update(z, dz, sr), dz)

    def final(x0, dz_list):
        x = x0
        for blk, dz in zip(model.blocks, dz_list):
            x = x + write(dz, blk.write.beta(dtype=dz.dtype))
        return x

    model.final_accumulate_reference = final
    return model


def model_train_steps(args, torch, dev):
    """The reference's training-step benchmark (bench/benchmark_lthc_v2.py:15-62) on this build: per model, bf16
    parameters in train mode, SGD(lr=0), images/targets [B,3,256,256] bf16 ~ N(0,1), t ~ U(0,1), labels uniform in
    [0,1000); one step = zero_grad, forward under bf16 autocast, fp32 MSE loss, backward, optimizer step; warm-up,
    then `model_steps` timed steps between two synchronisations (wall clock, as the reference times them).
    Models: the released lthc_b4_velocity and the v2 shared-AdaLN model (its triangular interface)."""
    import time

    from flowmatching_lthc_amd import model as M

    B = args.model_batch
    out = {}
    for name in ("lthc_b4_velocity", "local_thc_v2_fused_final12_shared_adaln_b4"):
        torch.manual_seed(123)
        model = M.build_model(name).to(device=dev, dtype=torch.bfloat16).train()
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        gen = torch.Generator(device=dev).manual_seed(3)
        x = torch.randn((B, 3, 256, 256), generator=gen, device=dev, dtype=torch.bfloat16)
        target = torch.randn((B, 3, 256, 256), generator=gen, device=dev, dtype=torch.bfloat16)
        t = torch.rand((B,), generator=gen, device=dev)
        y = torch.randint(0, 1000, (B,), generator=gen, device=dev)

        def step():
            opt.zero_grad(set_to_none=True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                pred = model(x, t, y)
                loss = (pred.float() - target.float()).square().mean()
            loss.backward()
            opt.step()
            return loss

        torch.cuda.reset_peak_memory_stats()
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.model_steps):
            loss = step()
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / args.model_steps
        out[name] = {
            "step_ms": round(step_s * 1e3, 3),
            "samples_per_s": round(B / step_s, 1),
            "peak_gib": round(torch.cuda.max_memory_allocated() / 2**30, 2),
            "loss": float(loss.detach()),
        }
        del model, opt, x, target
        torch.cuda.empty_cache()
    return {
        "workload": "training step as bench/benchmark_lthc_v2.py times it (bf16 parameters, autocast, MSE, SGD lr=0), eager",
        "batch": B,
        "steps": args.model_steps,
        "models": out,
    }


def model_forward(args, torch, dev, compare=True):
    """LTHC-B/4 forward, random-init weights, bf16 autocast, images [B,3,256,256] ~ N(0,1), t ~ U(0,1), labels
    uniform in [0,1000).  Timed eagerly and as one HIP graph replayed per forward (static inputs; the replay
    is checked bit-for-bit against the eager output), with fp32 parameters (the headline figure) and with
    bf16 parameters as the reference's benchmark holds the model, and -- with compare -- with the interface
    as torch eager ops for comparison."""
    from flowmatching_lthc_amd import model as M

    B = args.model_batch
    gen = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn((B, 3, 256, 256), generator=gen, device=dev)
    t = torch.rand((B,), generator=gen, device=dev)
    y = torch.randint(0, 1000, (B,), generator=gen, device=dev)
    stream = torch.cuda.current_stream()

    def timed(m):
        def fwd():
            with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
                return m(x, t, y)

        for _ in range(args.warmup):
            fwd()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.model_steps):
            out = fwd()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.model_steps, out

    def graphed(m, ref):
        def fwd():
            with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
                return m(x, t, y)

        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for _ in range(2):
                fwd()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = fwd()
        g.replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(out, ref))
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.model_steps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.model_steps
        del g, out
        return ms, same

    name = args.model_name
    ours = M.randomize_parameters(M.build_model(name), seed=0).to(dev).eval()
    ms, out_ours = timed(ours)
    ms_graph, graph_same = graphed(ours, out_ours)
    # bf16 parameters under autocast, as the reference's benchmark holds the model (bench/benchmark_lthc_v2.py:28):
    # no per-forward weight casts
    ours16 = M.randomize_parameters(M.build_model(name), seed=0).to(dev, torch.bfloat16).eval()
    ms16, out16 = timed(ours16)
    ms16_graph, graph16_same = graphed(ours16, out16)
    diff16 = float((out16.float() - out_ours.float()).abs().max() / out_ours.float().abs().max())
    del ours16
    res = {
        "img_per_s": round(B / (ms_graph * 1e-3), 1),
        "ms_per_fwd": round(ms_graph, 4),
        "timing": "one HIP graph per forward, replayed (eager launches below)",
        "graph_equals_eager": graph_same,
        "eager_img_per_s": round(B / (ms * 1e-3), 1),
        "eager_ms_per_fwd": round(ms, 4),
        "bf16_params_img_per_s": round(B / (ms16_graph * 1e-3), 1),
        "bf16_params_ms_per_fwd": round(ms16_graph, 4),
        "bf16_params_graph_equals_eager": graph16_same,
        "bf16_params_eager_img_per_s": round(B / (ms16 * 1e-3), 1),
        "bf16_params_max_rel_diff_vs_fp32_params": diff16,
        "batch": B,
        "steps": args.model_steps,
        "workload": f"{name} forward, random-init weights, bf16 autocast",
    }
    if compare and name == "lthc_b4_velocity":
        eager = eager_interface(M.randomize_parameters(M.build_model("lthc_b4_velocity"), seed=0).to(dev).eval(), torch)
        ms_eager, out_eager = timed(eager)
        res["torch_eager_interface_img_per_s"] = round(B / (ms_eager * 1e-3), 1)
        res["torch_eager_interface_ms_per_fwd"] = round(ms_eager, 4)
        res["max_rel_diff_vs_torch_eager_interface"] = float(
            (out_ours.float() - out_eager.float()).abs().max() / out_eager.float().abs().max()
        )
    return res


def interface_forward(args, torch, dev, ops, B, G, C, L):
    """The interface forward step (read, gamma stack, L recurrence steps, materialise) at one configuration,
    captured as a HIP graph per input set (two sets) and replayed; returns ms per step and GB/s of the per-op
    compulsory bytes."""
    H = 4 * G
    bf16 = torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(7)
    alpha = torch.randn((C, 16), generator=gen, device=dev) * 0.01 + 1.0 / 16.0
    beta_stack = torch.randn((L, C, 16), generator=gen, device=dev) * 0.02
    betas = list(beta_stack.unbind(0))
    sets = []
    for _ in range(2):
        x0 = torch.randn((B, H, H, C), generator=gen, device=dev).to(bf16)
        dzs = [(torch.randn((B, G * G, C), generator=gen, device=dev) * 0.02).to(bf16) for _ in range(L)]
        sets.append((x0, dzs))
    stream = torch.cuda.current_stream()

    def step(i):
        x0, dzs = sets[i % 2]
        z = ops.local_write_traceable(x0, alpha)
        gam = ops.lazy_gamma_stack(alpha, beta_stack)
        for l in range(L):
            z = ops.lazy_workspace_update(z, dzs[l], gam[l])
        if L == 12:
            xl = ops.final_accumulate_b4_12_traceable(x0, *dzs, *betas)
        else:
            xl = ops.final_accumulate_list(x0, dzs, betas)
        return z, xl

    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for i in range(2):
            step(i)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graphs = []
    for i in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(i)
        graphs.append(g)
    for i in range(max(2, args.warmup)):
        graphs[i % 2].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.steps):
        graphs[i % 2].replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = algorithmic_bytes(B, G, C, L)["total"]
    return {
        "B": B, "high_grid": H, "workspace_grid": G, "C": C, "L": L,
        "ms_per_step": round(ms, 4),
        "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "pct_of_peak_hbm": round(100.0 * nbytes / (ms * 1e-3) / PEAK_HBM, 2),
    }


def interface_c_level(args, torch, dev, B, G, C, L):
    """The whole-interface C entry points with every dZ_l given (lthc_interface_fwd, lthc_interface_bwd): one call
    each, no autograd, events around `steps` calls over two input sets.  Not the metric's step (the model's lazy
    forward runs a branch between the recurrence steps); reported beside it.  Bytes: forward e(2T + (2L + 1)W), the
    single-pass compulsory bytes (read X0 and the dZ stack; write X_L and Z_0 .. Z_L), which the one-pass kernel
    moves.  Backward: the single-pass compulsory bytes e(3T + 3LW) (read
    G_L, X0, the H and dZ stacks; write dX0 and the dZ-gradient stack), against which the rate is reported; the
    implementation moves e(3T + 3LW + 2W): the tile kernel e(2T + 3LW + W) (it also writes S_0) and dalpha's pass
    over X0 and S_0 e(T + W)."""
    from flowmatching_lthc_amd import _abi

    lib = _abi.load()
    H = 4 * G
    bf16 = torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(13)
    alpha = torch.randn((C, 16), generator=gen, device=dev) * 0.01 + 1.0 / 16.0
    betas = [torch.randn((C, 16), generator=gen, device=dev) * 0.02 for _ in range(L)]
    sets = []
    for _ in range(2):
        x0 = torch.randn((B, H, H, C), generator=gen, device=dev).to(bf16)
        dzs = [(torch.randn((B, G * G, C), generator=gen, device=dev) * 0.02).to(bf16) for _ in range(L)]
        sets.append((x0, dzs, _abi.ptr_array(dzs)))
    zs = [torch.empty((B, G * G, C), device=dev, dtype=bf16) for _ in range(L + 1)]
    xl = torch.empty((B, H, H, C), device=dev, dtype=bf16)
    nbytes = int(lib.lthc_interface_workspace_bytes(B, G, 4, C, L))
    ws = torch.empty((max(nbytes, 16),), device=dev, dtype=torch.uint8)
    stream = torch.cuda.current_stream()
    sid = stream.cuda_stream
    bp, zp = _abi.ptr_array(betas), _abi.ptr_array(zs)

    def fwd(i):
        x0, _, dzp = sets[i & 1]
        _abi.check(lib.lthc_interface_fwd(
            x0.data_ptr(), _abi.code(x0), alpha.data_ptr(), bp, _abi.code(alpha), dzp, zp, xl.data_ptr(), B, G, 4, C,
            L, ws.data_ptr(), ws.numel(), sid,
        ), "lthc_interface_fwd")  # fmt: skip

    gx = (torch.randn((B, H, H, C), generator=gen, device=dev) * 1e-3).to(bf16)
    gzs = [(torch.randn((B, G * G, C), generator=gen, device=dev) * 1e-3).to(bf16) for _ in range(L)]
    dx0 = torch.empty_like(gx)
    ddz = [torch.empty((B, G * G, C), device=dev, dtype=bf16) for _ in range(L)]
    da = torch.empty((C, 16), device=dev, dtype=torch.float32)
    db = torch.empty((L, C, 16), device=dev, dtype=torch.float32)
    gzp, ddzp = _abi.ptr_array(gzs), _abi.ptr_array(ddz)

    def bwd(i):
        x0, _, dzp = sets[i & 1]
        _abi.check(lib.lthc_interface_bwd(
            gx.data_ptr(), gzp, _abi.code(gx), x0.data_ptr(), dzp, alpha.data_ptr(), bp,
            _abi.code(alpha), dx0.data_ptr(), ddzp, da.data_ptr(), db.data_ptr(), B, G, 4, C, L,
            ws.data_ptr(), ws.numel(), sid,
        ), "lthc_interface_bwd")  # fmt: skip

    def timed(fn):
        for i in range(args.warmup):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(args.steps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    fwd_ms, bwd_ms = timed(fwd), timed(bwd)
    T, W = B * H * H * C, B * G * G * C
    fb = 2 * (2 * T + (2 * L + 1) * W)
    bb = 2 * (3 * T + 3 * L * W)
    out = {
        "workload": f"whole-interface C calls, every dZ_l given (B={B}, {H}x{H}/{G}x{G}, C={C}, L={L}, bf16, fp32 weights)",
        "timing": "events around consecutive calls, eager (several launches per call)",
        "fwd_ms": round(fwd_ms, 4),
        "fwd_bytes": fb,
        "fwd_byte_definition": "single-pass compulsory e(2T + (2L + 1)W): X0 and the dZ stack read once, X_L and Z_0..Z_L written",
        "fwd_GBps": round(fb / (fwd_ms * 1e-3) / 1e9, 1),
        "fwd_pct_of_peak_hbm": round(100.0 * fb / (fwd_ms * 1e-3) / PEAK_HBM, 2),
        "bwd_ms": round(bwd_ms, 4),
        "bwd_bytes": bb,
        "bwd_byte_definition": "single-pass compulsory e(3T + 3LW); the implementation moves e(3T + 3LW + 2W)",
        "bwd_GBps": round(bb / (bwd_ms * 1e-3) / 1e9, 1),
        "bwd_pct_of_peak_hbm": round(100.0 * bb / (bwd_ms * 1e-3) / PEAK_HBM, 2),
    }
    del sets, zs, xl, ws, gx, gzs, dx0, ddz
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def triangular_forward(args, torch, dev, B, G, C, L):
    """The non-shared (triangular lazy) interface forward at one shape: the L bases R_l(x0) in one pass
    (jit_thc::all_base_b4_12_split_traceable), the L-1 workspace sums z_l = base_l + sum_{j<l} gamma[l,j] dz_j
    (the active-prefix ops at depth 12, triangular_accumulate_list otherwise) and the materialisation, with
    synthetic dz_l standing in for the branch.  Graph-replayed over two input sets like interface_forward.
    Compulsory bytes: bases e(T + LW), sums e*sum_{l=1}^{L-1}(l+2)W, materialise e(2T + LW), plus weights."""
    from flowmatching_lthc_amd import ops
    from flowmatching_lthc_amd import ops_triangular as T

    H = 4 * G
    bf16 = torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(11)
    alpha_stack = (torch.randn((L, C, 16), generator=gen, device=dev) * 0.01 + 1.0 / 16.0).to(bf16)
    beta_stack = (torch.randn((L, C, 16), generator=gen, device=dev) * 0.02).to(bf16)
    betas = list(beta_stack.unbind(0))
    gamma = T.gamma_matrix(alpha_stack, beta_stack)
    sets = []
    for _ in range(2):
        x0 = torch.randn((B, H, H, C), generator=gen, device=dev).to(bf16)
        dzs = [(torch.randn((B, G * G, C), generator=gen, device=dev) * 0.02).to(bf16) for _ in range(L)]
        sets.append((x0, dzs))
    zero = torch.zeros_like(sets[0][1][0])
    stream = torch.cuda.current_stream()
    ws_events = []

    def step(i, timed=False):
        x0, dzs = sets[i % 2]
        bases = T.all_base_b4_12_split_traceable(x0, alpha_stack)
        if timed:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
        zs = [bases[0]]
        for l in range(1, L):
            if L == 12:
                args12 = tuple(dzs[j] if j < l else zero for j in range(12))
                zs.append(T.triangular_accumulate_b4_12_ptr_active_traceable_ops[l - 1](bases[l], *args12, gamma[l]))
            else:
                zs.append(T.triangular_accumulate_list(bases[l], dzs[:l], gamma[l, :l].contiguous()))
        if timed:
            e1.record(stream)
            ws_events.append((e0, e1))
        xl = ops.final_accumulate_list(x0, dzs, betas)
        return zs, xl

    for i in range(max(2, args.warmup)):
        step(i, timed=True)
    torch.cuda.synchronize()
    ws_events.clear()
    for i in range(args.steps):
        step(i, timed=True)
    torch.cuda.synchronize()
    ws_ms = sum(a.elapsed_time(b) for a, b in ws_events) / len(ws_events)

    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for i in range(2):
            step(i)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    graphs, outs = [], []
    for i in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs.append(step(i))
        graphs.append(g)
    ref = step(0)
    graphs[0].replay()
    torch.cuda.synchronize()
    same = torch.equal(outs[0][1], ref[1]) and all(torch.equal(a, b) for a, b in zip(outs[0][0], ref[0]))
    for i in range(max(2, args.warmup)):
        graphs[i % 2].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.steps):
        graphs[i % 2].replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    e, T_, W = 2, B * H * H * C, B * G * G * C
    wbytes = 2 * 16 * C * L
    by = {
        "bases": e * (T_ + L * W) + wbytes,
        "triangular_sums": sum(e * (l + 2) * W + e * l * C for l in range(1, L)),
        "materialise": e * (2 * T_ + L * W) + wbytes,
    }
    total = sum(by.values())
    del sets, graphs, outs, ref
    return {
        "B": B, "high_grid": H, "workspace_grid": G, "C": C, "L": L,
        "ms_per_step": round(ms, 4),
        "GBps": round(total / (ms * 1e-3) / 1e9, 1),
        "pct_of_peak_hbm": round(100.0 * total / (ms * 1e-3) / PEAK_HBM, 2),
        "triangular_sums_ms_eager": round(ws_ms, 4),
        "triangular_sums_GBps": round(by["triangular_sums"] / (ws_ms * 1e-3) / 1e9, 1),
        "bytes_by_op": by,
        "graph_equals_eager": same,
    }  # fmt: skip


def interface_train(args, torch, dev, ops, B=None, G=None, C=None, L=None, label="configuration 3"):
    """Benchmark configuration 3: the interface forward + autograd backward at the training shape (B=64, bf16).

    X0, alpha, the 12 beta_l and the 12 dZ_l are leaves that require grad; the upstream gradients are
    G_L = dL/dX_L ~ N(0, 1e-3) and H_l = dL/dZ_l ~ N(0, 1e-3) for the 12 workspace states Z_0..Z_11 that feed
    the branches.  One step = read (the fused-open form of the model's forward_lazy), every gamma (one launch), 12
    recurrence steps, 12-pointer materialise, then torch.autograd.grad over (X_L, Z_0..Z_11) -- every backward
    kernel of the interface plus autograd's own gradient accumulation (adds), as in training."""
    B = args.train_batch if B is None else B
    G = args.grid if G is None else G
    C = args.channels if C is None else C
    L = args.depth if L is None else L
    H = 4 * G
    bf16 = torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(3)
    x0 = torch.randn((B, H, H, C), generator=gen, device=dev).to(bf16).requires_grad_()
    alpha = (torch.randn((C, 16), generator=gen, device=dev) * 0.01 + 1.0 / 16.0).requires_grad_()
    betas = [(torch.randn((C, 16), generator=gen, device=dev) * 0.02).requires_grad_() for _ in range(L)]
    dzs = [(torch.randn((B, G * G, C), generator=gen, device=dev) * 0.02).to(bf16).requires_grad_() for _ in range(L)]
    g_out = (torch.randn((B, H, H, C), generator=gen, device=dev) * 1e-3).to(bf16)
    h_ws = [(torch.randn((B, G * G, C), generator=gen, device=dev) * 1e-3).to(bf16) for _ in range(L)]
    stream = torch.cuda.current_stream()

    def forward():
        x0v, z = ops.read_with_residual(x0, alpha.to(bf16))  # as the model's forward_lazy
        # every layer's gamma_from_alpha in one launch, as the model's forward_lazy; the rows as one unbind (its
        # backward is one stack, not a zero-fill + copy + add per layer)
        gam = ops.lazy_gamma_rounded(alpha, betas, bf16).unbind(0)
        zs, dzv = [z], []
        for l in range(L):
            z, zb, d = ops.lazy_workspace_step(z, dzs[l], gam[l], split=True)  # as the model's forward_lazy
            zs.append(zb)  # the next branch's input
            dzv.append(d)
        if L == 12:
            xl = ops.final_accumulate_b4_12_traceable(x0v, *dzv, *betas)
        else:  # the base-class materialisation of the model (list op)
            xl = ops.final_accumulate_list(x0v, dzv, betas)
        return xl, zs[:L]

    leaves = [x0, alpha] + betas + dzs

    def step():
        xl, zs = forward()
        return torch.autograd.grad([xl] + zs, leaves, [g_out] + h_ws)

    def fwd_only():
        with torch.no_grad():
            return forward()

    def timed(fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    eager_fwd = timed(fwd_only)
    eager_step = timed(step)

    # HIP graphs of the forward alone and of forward + backward, replayed
    graph_fwd = graph_step = None
    graph_error = None
    try:
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for _ in range(3):
                step()
                fwd_only()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        g_fwd, g_step = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_fwd):
            fwd_only()
        with torch.cuda.graph(g_step):
            grads_graph = step()
        grads_eager = step()
        g_step.replay()
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(grads_graph, grads_eager)):
            raise RuntimeError("graph replay of the training step differs from the eager step")
        graph_fwd = timed(g_fwd.replay)
        graph_step = timed(g_step.replay)
    except RuntimeError as exc:  # report the eager timing with the reason
        graph_error = str(exc)[:300]
        torch.cuda.synchronize()
    T = B * H * H * C
    W = B * G * G * C
    fused_bwd = 2 * (3 * T + 3 * L * W)
    # per-op compulsory bytes: materialise backward e(T + 2LW) (gdZ and gbeta from one read of G_L: the tile kernel
    # mbwd_mfma_kernel), recurrence backward e(6LW) (per layer g, dz, the branch gradient and the materialisation's
    # gradient in, two out), read backward e(3T + W) (G_L, gZ0 and X0 in, dX0 out)
    per_op_bwd = 2 * (4 * T + 8 * L * W + W)
    fwd_ms, step_ms = (graph_fwd, graph_step) if graph_error is None else (eager_fwd, eager_step)
    bwd_ms = step_ms - fwd_ms
    return {
        "workload": f"interface fwd + autograd bwd, {label} (B={B}, {H}x{H}/{G}x{G}, C={C}, L={L}, bf16, fp32 weights)",
        "batch": B,
        "steps": args.steps,
        "timing": "HIP graph replays (forward alone; forward + autograd.grad), eager for comparison"
        if graph_error is None
        else f"eager (graph capture failed: {graph_error})",
        "fwd_ms": round(fwd_ms, 4),
        "fwd_bwd_ms": round(step_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "eager_fwd_ms": round(eager_fwd, 4),
        "eager_fwd_bwd_ms": round(eager_step, 4),
        "bwd_single_pass_bytes": fused_bwd,
        "bwd_single_pass_GBps": round(fused_bwd / (bwd_ms * 1e-3) / 1e9, 1),
        "bwd_per_op_bytes": per_op_bwd,
        "bwd_per_op_GBps": round(per_op_bwd / (bwd_ms * 1e-3) / 1e9, 1),
        "byte_definition": "bwd_single_pass_bytes = e*(3T + 3LW): the compulsory bytes of a fused single-pass backward "
        "(read G_L, X0, H stack, dZ stack; write dX0, dZ-grad stack); bwd_per_op_bytes = e*(4T + 8LW + W): each "
        "backward op's compulsory bytes (materialise e(T+2LW), L recurrence steps e(6LW), read e(3T+W)); autograd "
        "runs these ops, so G_L is read twice (materialise backward, read backward)",
    }


def recurrence_cache_leg(args, torch, ops, sets, alpha, beta_stack, L, W, step_ms, step_bytes):
    """The step's L recurrence launches timed one by one with events: as they run in the step (Z_l written by the
    previous launch just before), with Z_l and dZ_l evicted from the 256 MB MALL by an untimed 1 GiB read sweep
    before each launch (both then come from HBM), and after an untimed 1 GiB streaming fill instead (the same
    eviction, plus the fill's dirty lines written back while the launch runs).  Reports the three rates and the step
    time each cold form implies: step_ms + sum_l (cold_l - in_step_l)."""
    stream = torch.cuda.current_stream()
    sweep = torch.ones((1 << 30) // 4, device=sets[0][0].device, dtype=torch.float32)
    sink = torch.zeros((), device=sweep.device, dtype=torch.float32)
    reps = max(2, min(args.steps, 10))

    def run(evict):
        ev = []
        for i in range(reps):
            x0, dzs = sets[i % 2]
            z = ops.local_write_traceable(x0, alpha)
            gam = ops.lazy_gamma_stack(alpha, beta_stack)
            for l in range(L):
                if evict == "read":
                    sink.add_(sweep.sum())
                elif evict == "write":
                    sweep.fill_(float(l))
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                z = ops.lazy_workspace_update(z, dzs[l], gam[l])
                e1.record(stream)
                ev.append((e0, e1))
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in ev) / len(ev)

    run("read")  # warm-up of every path
    run("write")
    warm_ms, read_ms, write_ms = run(None), run("read"), run("write")
    del sweep
    rb = 2 * 3 * W  # bytes per launch: Z_l and dZ_l in, Z_{l+1} out (bf16; gamma negligible)

    def implied(ms):
        step = step_ms + L * (ms - warm_ms)
        return round(step, 4), round(100.0 * step_bytes / (step * 1e-3) / PEAK_HBM, 2)

    read_step, read_pct = implied(read_ms)
    write_step, write_pct = implied(write_ms)
    return {
        "per_launch_us_in_step_order": round(warm_ms * 1e3, 2),
        "per_launch_GBps_in_step_order": round(rb / (warm_ms * 1e-3) / 1e9, 1),
        "per_launch_us_hbm_cold": round(read_ms * 1e3, 2),
        "per_launch_GBps_hbm_cold": round(rb / (read_ms * 1e-3) / 1e9, 1),
        "step_ms_implied_hbm_cold": read_step,
        "pct_of_peak_hbm_implied_hbm_cold": read_pct,
        "per_launch_us_after_write_fill": round(write_ms * 1e3, 2),
        "per_launch_GBps_after_write_fill": round(rb / (write_ms * 1e-3) / 1e9, 1),
        "step_ms_implied_after_write_fill": write_step,
        "pct_of_peak_hbm_implied_after_write_fill": write_pct,
        "note": "the headline value times the step as launched back to back, where each recurrence launch reads the "
        "Z_l that the previous launch wrote microseconds earlier; hbm_cold evicts Z_l and dZ_l with a 1 GiB read "
        "sweep before every launch (both then come from HBM); after_write_fill evicts them with a 1 GiB fill, whose "
        "dirty lines are written back to HBM during the launch",
    }


def profile(args, ops, inputs, alpha, beta_stack, betas):
    """One kernel, --warmup + --steps launches, then a plain copy of X0 (bytes known: 2 x X0)."""
    import torch

    x0, dzs = inputs
    z = ops.local_write_traceable(x0, alpha)
    gam = ops.lazy_gamma_stack(alpha, beta_stack)
    if args.profile in ("mat_bwd", "interface_bwd", "interface_fwd"):
        import ctypes

        from flowmatching_lthc_amd import _abi

        lib = _abi.load()
        B, H, C = x0.shape[0], x0.shape[1], x0.shape[3]
        G, L = H // 4, len(dzs)
        sid = torch.cuda.current_stream().cuda_stream
        gdz = [torch.empty_like(d) for d in dzs]
        gb = torch.empty((L, C, 16), device=x0.device)
        if args.profile == "mat_bwd":  # G_L = x0's values (the data do not change the traffic)
            ws = torch.empty((int(lib.lthc_materialise_bwd_workspace_bytes(B, G, 4, C, L)),), device=x0.device,
                             dtype=torch.uint8)  # fmt: skip

            def run():
                _abi.check(lib.lthc_materialise_bwd(
                    x0.data_ptr(), _abi.code(x0), _abi.ptr_array(dzs), _abi.ptr_array(betas), _abi.code(alpha),
                    _abi.ptr_array(gdz), gb.data_ptr(), B, G, 4, C, L, ws.data_ptr(), ws.numel(), sid,
                ), "lthc_materialise_bwd")  # fmt: skip
        elif args.profile == "interface_fwd":
            ws = torch.empty((int(lib.lthc_interface_workspace_bytes(B, G, 4, C, L)),), device=x0.device,
                             dtype=torch.uint8)  # fmt: skip
            zs = [torch.empty_like(dzs[0]) for _ in range(L + 1)]
            xl = torch.empty_like(x0)

            def run():
                _abi.check(lib.lthc_interface_fwd(
                    x0.data_ptr(), _abi.code(x0), alpha.data_ptr(), _abi.ptr_array(betas), _abi.code(alpha),
                    _abi.ptr_array(dzs), _abi.ptr_array(zs), xl.data_ptr(), B, G, 4, C, L, ws.data_ptr(),
                    ws.numel(), sid,
                ), "lthc_interface_fwd")  # fmt: skip
        else:  # G_L = x0; H_l tensors of their own (aliasing dZ_l would serve them from cache)
            ws = torch.empty((int(lib.lthc_interface_workspace_bytes(B, G, 4, C, L)),), device=x0.device,
                             dtype=torch.uint8)  # fmt: skip
            dx0 = torch.empty_like(x0)
            da = torch.empty((C, 16), device=x0.device)
            hs = [d * 0.5 for d in dzs]
            gz = (ctypes.c_void_p * L)(*[h.data_ptr() for h in hs])

            def run():
                _abi.check(lib.lthc_interface_bwd(
                    x0.data_ptr(), gz, _abi.code(x0), x0.data_ptr(), _abi.ptr_array(dzs), alpha.data_ptr(),
                    _abi.ptr_array(betas), _abi.code(alpha), dx0.data_ptr(), _abi.ptr_array(gdz), da.data_ptr(),
                    gb.data_ptr(), B, G, 4, C, L, ws.data_ptr(), ws.numel(), sid,
                ), "lthc_interface_bwd")  # fmt: skip
        for _ in range(args.warmup + args.steps):
            run()
        torch.cuda.synchronize()
        y = torch.empty_like(x0)
        y.copy_(x0)
        torch.cuda.synchronize()
        print(f"profiled {args.profile} x{args.warmup + args.steps}; calibration copy of {x0.numel() * x0.element_size()} bytes")
        return
    run = {
        # the depth-12 op of the reference at depth 12, the list op (any depth) otherwise
        "materialise": (lambda: ops.final_accumulate_b4_12_traceable(x0, *dzs, *betas))
        if len(dzs) == 12
        else (lambda: ops.final_accumulate_list(x0, dzs, betas)),
        "read": lambda: ops.local_write_traceable(x0, alpha),
        "recur": lambda: ops.lazy_workspace_update(z, dzs[0], gam[0]),
        "read_multi": lambda: ops.final_accumulate_b4_12_grad_dz_ptr_traceable(x0, *betas),
        "weight_grad": lambda: ops.final_accumulate_b4_12_grad_beta_ptr_traceable(x0, *dzs),
        "copy": lambda: None,
    }[args.profile]
    for _ in range(args.warmup + args.steps):
        run()
    torch.cuda.synchronize()
    y = torch.empty_like(x0)
    y.copy_(x0)
    torch.cuda.synchronize()
    print(f"profiled {args.profile} x{args.warmup + args.steps}; calibration copy of {x0.numel() * x0.element_size()} bytes")


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (the interface would shard along "
            "the batch: each GPU runs the same kernels on B/N samples and the weight gradients join the data-parallel "
            "all-reduce)",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    sys.path.insert(0, ROOT)
    from flowmatching_lthc_amd import ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (torch.cuda.is_available() is False)", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.profile == "model":
        print(json.dumps({"model_fwd": model_forward(args, torch, dev, compare=False)}))
        return
    if args.profile == "train":
        print(json.dumps({"interface_train": interface_train(args, torch, dev, ops)}))
        return
    if args.profile == "interface_c":  # the whole-interface C calls at the training batch (configuration 3)
        leg = interface_c_level(args, torch, dev, args.train_batch, args.grid, args.channels, args.depth)
        print(json.dumps({"interface_c_level": leg}))
        return
    if args.profile == "triangular":
        tri = triangular_forward(args, torch, dev, args.batch, args.grid, args.channels, args.depth)
        print(json.dumps({"triangular_fwd": tri}))
        return
    B, G, C, L = args.batch, args.grid, args.channels, args.depth
    H = 4 * G
    bf16 = torch.bfloat16

    gen = torch.Generator(device=dev).manual_seed(0)

    def make_set():
        x0 = torch.randn((B, H, H, C), generator=gen, device=dev).to(bf16)
        dzs = [(torch.randn((B, G * G, C), generator=gen, device=dev) * 0.02).to(bf16) for _ in range(L)]
        return x0, dzs

    alpha = torch.randn((C, 16), generator=gen, device=dev) * 0.01 + 1.0 / 16.0
    beta_stack = torch.randn((L, C, 16), generator=gen, device=dev) * 0.02
    betas = list(beta_stack.unbind(0))
    sets = [make_set(), make_set()]  # rotate two input sets so the 256 MB MALL cannot serve repeats
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    mat_events = []

    def step(i, timed=False):
        x0, dzs = sets[i % 2]
        z = ops.local_write_traceable(x0, alpha)
        gam = ops.lazy_gamma_stack(alpha, beta_stack)
        for l in range(L):
            z = ops.lazy_workspace_update(z, dzs[l], gam[l])
        if timed:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
        if L == 12:
            xl = ops.final_accumulate_b4_12_traceable(x0, *dzs, *betas)
        else:  # the layers as a list (no dz stack copy), as the model's generic materialisation
            xl = ops.final_accumulate_list(x0, dzs, betas)
        if timed:
            e1.record(stream)
            mat_events.append((e0, e1))
        return z, xl

    if args.profile:
        profile(args, ops, sets[0], alpha, beta_stack, betas)
        return

    # eager: warmup, then K timed steps with events around every materialise launch
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(args.steps):
        step(i, timed=True)
    t1.record(stream)
    torch.cuda.synchronize()
    eager_ms = t0.elapsed_time(t1) / args.steps
    mat_ms = sum(a.elapsed_time(b) for a, b in mat_events) / len(mat_events)

    # graph: one captured step per input set, replayed
    graph_ms = None
    graphs = []
    if args.mode == "graph":
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(2):
                step(i)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        outs = []
        for i in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                outs.append(step(i))
            graphs.append(g)
        ref = step(0)
        for i in range(max(2, args.warmup)):
            graphs[i % 2].replay()
        torch.cuda.synchronize()
        graphs[0].replay()
        torch.cuda.synchronize()
        if not (torch.equal(outs[0][1], ref[1]) and torch.equal(outs[0][0], ref[0])):
            print("graph replay differs from the eager step", file=sys.stderr)
            sys.exit(3)
        t0.record(stream)
        for i in range(args.steps):
            graphs[i % 2].replay()
        t1.record(stream)
        torch.cuda.synchronize()
        graph_ms = t0.elapsed_time(t1) / args.steps

    ms = graph_ms if graph_ms is not None else eager_ms
    nbytes = algorithmic_bytes(B, G, C, L)
    value = nbytes["total"] / (ms * 1e-3) / 1e9
    mat_achieved = nbytes["materialise"] / (mat_ms * 1e-3)
    traffic, traffic_source = pmc_traffic()
    recur_cache = recurrence_cache_leg(args, torch, ops, sets, alpha, beta_stack, L, B * G * G * C, ms, nbytes["total"])

    # release every tensor and graph pool of the main measurement before the other legs
    outs = ref = None
    del sets, graphs, outs, ref, mat_events
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    model_fwd = None if args.no_model else model_forward(args, torch, dev)
    model_train = None if args.no_model else model_train_steps(args, torch, dev)
    train = None if args.no_train else interface_train(args, torch, dev, ops)
    configs = None
    if not args.no_configs:
        configs = {
            "config2_fwd": interface_forward(args, torch, dev, ops, 32, 16, 768, 12),
            "config5_fwd": interface_forward(args, torch, dev, ops, 32, 32, 1024, 24),
            "config5_train": interface_train(args, torch, dev, ops, 32, 32, 1024, 24, label="configuration 5"),
            "triangular_fwd_metric_shape": triangular_forward(args, torch, dev, B, G, C, L),
            "interface_c_level_metric_shape": interface_c_level(args, torch, dev, B, G, C, L),
            "interface_c_level_config3": interface_c_level(args, torch, dev, args.train_batch, G, C, L),
            "interface_c_level_config5": interface_c_level(args, torch, dev, 32, 32, 1024, 24),
        }

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(B, G, C, L, args.cpu_seconds)
        cpu["c_oracle"] = c_oracle_baseline(G, C, L, max(2.0, args.cpu_seconds / 4))

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "lthc_interface_fwd (read + gamma + L recurrence steps + materialise)",
            "B": B,
            "high_grid": H,
            "workspace_grid": G,
            "C": C,
            "L": L,
            "weights": "fp32",
            "timing": f"{args.mode} ({'one HIP graph per step' if args.mode == 'graph' else 'eager op launches'})",
            "bytes_per_step": nbytes["total"],
            "byte_definition": "per-op compulsory: e*(3T+(4L+1)W) + weights, e=2",
            "pct_of_peak_hbm": round(100.0 * value * 1e9 / PEAK_HBM, 2),
        },
        "roofline": {
            "kernel": f"cell_mat_kernel<bf16 x, fp32 w, L={L}> (jit_thc::final_accumulate_{'b4_12_traceable' if L == 12 else 'list'})",
            "bound": "hbm",
            "achieved": round(mat_achieved / 1e9, 2),
            "peak": PEAK_HBM / 1e9,
            "unit": "GB/s",
            "frac": round(mat_achieved / PEAK_HBM, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes_per_launch": nbytes["materialise"],
            "avg_launch_ms": round(mat_ms, 4),
        },
        "cpu_baseline": cpu,
        "recurrence_mall": recur_cache,
        "model_fwd": model_fwd,
        "model_train": model_train,
        "interface_train": train,
        "configs": configs,
        "extra": {
            "eager_ms_per_step": round(eager_ms, 4),
            "graph_ms_per_step": None if graph_ms is None else round(graph_ms, 4),
            "bytes_by_op": nbytes,
            "device": torch.cuda.get_device_name(0),
        },
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
