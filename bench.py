"""Benchmark of the MI355X PAM hot path (one JSON line on stdout).

Workload ("config 2"): PAM chunked dual-form
prefill forward, fp32 complex planar, B=8, T=2048, H=12, d=64, C=64.  A step
is one scan forward over the whole batch (16384 tokens); `value` is tokens/s
with inputs resident in HBM.  `roofline` covers the dominant kernel (the
chunk-output MFMA kernel), timed live with HIP events recorded by the library
on the launch stream around that kernel, against the fp32 MFMA peak.

`roofline.frac_causal` counts the score and intra-read products over the
causal half of each chunk only; `traffic` (HBM bytes per launch) comes from
profiles/traffic.json, whose `build` hash is reported beside the current one.

Secondary measurements (same line, under "extras"): config 4 ragged decode
(256 slots, ~75% active, 1000 steps) in tokens/s and HBM GB/s, the E3 decode
engine, config 3 E3 fwd+bwd, config 5 CE fwd+bwd, complex elementwise ops,
the fused layer and the E2 delta rule.  `cpu_baseline` times the CPU
restatement of the reference's chunk loop (oracle/pam.py: chunked_head) on a
bounded sample of the same workload on the host cores; `cpu_baselines` does
the same for configs 3, 4 and 5 (oracle restatements, bounded samples, with
the host's CPU model and torch version).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu]
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_FP32_PEAK = 157.3e12
MFMA_BF16_PEAK = 2516.6e12
HBM_PEAK = 8.0e12


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--only", choices=["scan_fwd", "decode", "decode_e3", "engine", "model", "e3", "ce", "cplx", "layer",
                                       "delta", "delta_ref", "e1", "copy"], default=None,
                    help="run one workload (for profiler passes) and print its own JSON line")
    return ap.parse_args()


def source_hash():
    """16 hex digits of the SHA-256 of the library's sources (every .hip / .h
    under qllm2_amd/csrc and include/qpam.h, in name order): the build a
    measurement belongs to."""
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "qllm2_amd", "csrc")
    files = sorted(os.path.join(csrc, f) for f in os.listdir(csrc) if f.endswith((".hip", ".h")))
    for path in files + [os.path.join(ROOT, "include", "qpam.h")]:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(kernel_key):
    """(HBM bytes per dispatch of `kernel_key`, build hash of that measurement)
    from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (profiles/traffic.json, calibrated against a plain copy); bytes None when
    that kernel has not been measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        return None, None
    entry = doc.get("kernels", {}).get(kernel_key)
    return (entry["hbm_bytes"] if entry else None), doc.get("build")


def cpu_threads():
    """Threads for the CPU baselines: the CPUs this process may run on, capped
    at OMP_NUM_THREADS when it is set (the GPU boxes set it to their CPU share)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def host_info(threads):
    import platform
    import torch
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cores": threads, "host_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "cpu_model": model, "torch": torch.__version__}


def copy_calibration(nbytes=1 << 30, reps=3):
    """A plain device copy of known size: the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters into HBM bytes."""
    import torch
    src = torch.ones(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes_each_way": nbytes, "reps": reps}


def scan_inputs(B, H, T, d, M, seed, dtype, unit_qk=True, mu=3.0, mu_step=0.0):
    import torch
    from oracle.pam import make_scan_inputs
    q, k, v, gamma = make_scan_inputs(B, H, T, d, seed, m_states=M, unit_qk=unit_qk, gamma_mu=mu,
                                      gamma_mu_step=mu_step, dtype=torch.float32)
    dev = torch.device("cuda")

    def planes(x):
        return x[..., 0].contiguous().to(dtype).to(dev), x[..., 1].contiguous().to(dtype).to(dev)

    return planes(q), planes(k), planes(v), gamma.to(dev)


def bench_scan_fwd(steps, warmup):
    """Config 2: fp32 scan forward.  Returns (ms_per_step, kernel_ms, tokens)."""
    import torch
    from qllm2_amd import _lib, pam_scan
    from oracle.pam import scan_flops
    B, H, T, d, C = 8, 12, 2048, 64, 64
    (qr, qi), (kr, ki), (vr, vi), gamma = scan_inputs(B, H, T, d, 1, 1002, torch.float32)

    def step():
        return pam_scan.scan_fwd_op(qr, qi, kr, ki, vr, vi, gamma, None, None, None, None, d ** -0.5, C, 0)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    pairs = [_lib.EventPair() for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        pam_scan.set_profile_events(pairs[i])
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    kms = statistics.mean(p.elapsed_ms() for p in pairs)
    # dominant kernel algorithmic FLOPs: score + intra read + carried read (3 of the 4
    # per-chunk complex GEMMs; the state write runs in chunk_state_kernel), carried
    # read skipped on chunk 0
    n = math.ceil(T / C)
    kflops = B * H * (n * (8 * C * C * d * 2) + (n - 1) * 8 * C * d * d)
    # the same with the score and intra read counted over the causal half (C (C + 1) / 2 of C^2 pairs)
    kflops_causal = B * H * (n * (8 * (C * (C + 1) // 2) * d * 2) + (n - 1) * 8 * C * d * d)
    return dt * 1e3, kms, B * T, scan_flops(B, H, T, d, C), kflops, kflops_causal


def bench_decode(n_steps):
    """Config 4: ragged decode over 256 slots x 16 layers x 12 heads, d=64."""
    import torch
    from qllm2_amd.decode import decode_step
    S, L, H, d = 256, 16, 12, 64
    G = L * H
    dev = torch.device("cuda")
    gen = torch.Generator().manual_seed(1004)
    state = torch.empty(S, G, 1, d, d, 2, device=dev)
    for sl in range(0, S, 32):  # fill in pieces to bound host memory
        state[sl:sl + 32] = (torch.randn(32, G, 1, d, d, 2, generator=gen) * 0.01).to(dev)
    q, k, v = (torch.randn(S, G, d, 2, generator=gen).to(dev) for _ in range(3))
    gamma = torch.sigmoid(torch.randn(S, G, 1, generator=gen) + 3).to(dev)
    masks = [torch.nonzero(torch.rand(S, generator=gen) < 0.75).flatten().to(torch.int32).to(dev)
             for _ in range(16)]
    counts = [int(m.numel()) for m in masks]
    y = torch.zeros_like(q)
    for i in range(20):
        decode_step(state, q, k, v, gamma, active=masks[i % 16], q_scale=d ** -0.5, out=y)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n_steps):
        decode_step(state, q, k, v, gamma, active=masks[i % 16], q_scale=d ** -0.5, out=y)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n_steps
    active = sum(counts[i % 16] for i in range(n_steps)) / n_steps
    bytes_step = active * G * (2 * 32768 + 4 * 512 + 4)
    return {"ms_per_step": ms, "tokens_per_s": active / (ms * 1e-3), "active_slots": active,
            "hbm_GBps": bytes_step / (ms * 1e-3) / 1e9, "hbm_frac": bytes_step / (ms * 1e-3) / HBM_PEAK,
            "bytes_per_step": bytes_step, "steps": n_steps}


def bench_decode_e3_rope(n_steps):
    """Continuous-batching decode of an E3 model: 256 slots x 16 layers x 12 heads,
    3 states per head with per-state read rotation, d=64, per-slot RoPE positions,
    ~75% of slots active per step (one launch per step for all layers)."""
    import torch
    from qllm2_amd.decode import build_rope_cache, decode_step
    S, L, H, M, d = 256, 16, 12, 3, 64
    G = L * H
    dev = torch.device("cuda")
    gen = torch.Generator().manual_seed(1014)
    state = torch.empty(S, G, M, d, d, 2, device=dev)
    for sl in range(0, S, 16):
        state[sl:sl + 16] = (torch.randn(16, G, M, d, d, 2, generator=gen) * 0.01).to(dev)
    q, k, v = (torch.randn(S, G, d, 2, generator=gen).to(dev) for _ in range(3))
    gamma = torch.sigmoid(torch.randn(S, G, M, generator=gen) + 3).to(dev)
    rot = torch.randn(S, G, M, 2, generator=gen).to(dev)
    rope = build_rope_cache(8192, d, device=dev)
    pos = torch.randint(0, 8192, (S,), generator=gen, dtype=torch.int32).to(dev)
    masks = [torch.nonzero(torch.rand(S, generator=gen) < 0.75).flatten().to(torch.int32).to(dev)
             for _ in range(16)]
    counts = [int(m.numel()) for m in masks]
    y = torch.zeros_like(q)

    def step(i):
        decode_step(state, q, k, v, gamma, active=masks[i % 16], rot=rot, q_scale=d ** -0.5, out=y,
                    rope=rope, pos=pos)

    for i in range(10):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n_steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n_steps
    active = sum(counts[i % 16] for i in range(n_steps)) / n_steps
    # per active (slot, group): M states read+written (2 x 32 KiB each), q, k, v, y
    # rows (4 x 512 B), gamma + rotation per state (12 B); one rope row per slot
    bytes_step = active * G * (M * 2 * 32768 + 4 * 512 + M * 12) + active * 512
    return {"ms_per_step": ms, "tokens_per_s": active / (ms * 1e-3), "active_slots": active,
            "hbm_GBps": bytes_step / (ms * 1e-3) / 1e9, "hbm_frac": bytes_step / (ms * 1e-3) / HBM_PEAK,
            "bytes_per_step": bytes_step, "steps": n_steps}


def bench_engine(steps, warmup, graphs=False, dtype="fp32"):
    """Model-level continuous-batching decode (qllm2_amd.engine.DecodeEngine):
    16 E3 PAM layers (M=3, H=12, d=64, dim=768, fp32, RoPE, GSP, phase-routed
    states) over 256 slots, ~75% of them live per step.  A step runs every
    layer on the live rows: projection GEMM, gate GEMMs, the prologue kernel,
    one decode launch with per-slot RoPE, the o_proj GEMM.  With `graphs` the
    steps replay HIP graphs (one per live-count bucket of 16 rows); the warmup
    then runs every live set once, so every bucket is captured before timing."""
    import torch
    from qllm2_amd.engine import DecodeEngine
    S, L, H, d, M, dim = 256, 16, 12, 64, 3, 768
    layers = [_BenchPamLayer(dim, H, d, M, 16, torch.float32, seed=40 + i).mod for i in range(L)]
    engine = DecodeEngine(layers, n_slots=S, max_len=8192, graphs=graphs, graph_bucket=16,
                          dtype=torch.bfloat16 if dtype == "bf16" else torch.float32)
    if graphs:
        warmup = max(warmup, 16)
    gen = torch.Generator().manual_seed(1015)
    for s_ in range(S):
        engine.admit(int(torch.randint(1, 4096, (1,), generator=gen)))
    engine.pool.state.normal_(0.0, 0.01, generator=torch.Generator(device="cuda").manual_seed(1016))
    hosts = [torch.nonzero(torch.rand(S, generator=gen) < 0.75).flatten().tolist() for _ in range(16)]
    masks = [torch.tensor(h, dtype=torch.int32).cuda() for h in hosts]
    xs = [torch.randn(len(h), dim, 2, generator=gen).cuda() for h in hosts]

    def step(i):
        engine.step(xs[i % 16], masks[i % 16], host_slots=hosts[i % 16])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    active = sum(len(hosts[i % 16]) for i in range(steps)) / steps
    return {"config": f"16 PAM layers E3 M=3, H=12, d=64, dim=768, {dtype} GEMMs, 256 slots (~75% live)"
            + (", HIP-graph replay per live-count bucket of 16" if graphs else ""),
            "ms_per_step": ms, "tokens_per_s": active / (ms * 1e-3), "active_slots": active, "steps": steps}


def _bench_model(L, dim, H, d, M, vocab, expand, seed=70):
    """A V11LM-shaped module (the reference's attribute names) with random
    weights: L blocks of ComplexNorm, a ModSwish CGU of hidden expand * dim,
    the production E3 PAM layer of _BenchPamLayer; the tied embedding table,
    output norm, LM-head projection and norm."""
    import torch
    g = torch.Generator().manual_seed(seed)

    def prm(*shape, std, mean=0.0):
        return torch.nn.Parameter((torch.randn(*shape, generator=g) * std + mean).cuda())

    def clin(o, i, bias=False):
        lin = torch.nn.Module()
        lin.weight_real, lin.weight_imag = prm(o, i, std=(2 * i) ** -0.5), prm(o, i, std=(2 * i) ** -0.5)
        lin.bias_real = prm(o, std=0.02) if bias else None
        lin.bias_imag = prm(o, std=0.02) if bias else None
        return lin

    def norm(n):
        m = torch.nn.Module()
        m.scale, m.eps = prm(n, std=0.05, mean=1.0), 1e-6
        return m

    hid = expand * dim
    model = torch.nn.Module()
    model.embed = torch.nn.Module()
    for part in ("embed_real", "embed_imag"):
        e = torch.nn.Module()
        e.weight = prm(vocab, dim, std=0.02)
        setattr(model.embed, part, e)
    model.pos_embed = None
    model.embed_norm, model.output_norm, model.lm_head_norm = norm(dim), norm(dim), norm(dim)
    model.lm_head_proj = clin(dim, dim, bias=True)
    blocks = []
    for i in range(L):
        b = torch.nn.Module()
        b.norm1, b.norm2 = norm(dim), norm(dim)
        b.cgu = torch.nn.Module()
        b.cgu.gate_proj, b.cgu.up_proj, b.cgu.down_proj = clin(hid, dim), clin(hid, dim), clin(dim, hid)
        b.cgu.act = torch.nn.Module()
        b.cgu.act.bias, b.cgu.act.beta = prm(hid, std=0.1), prm(hid, std=0.1, mean=1.0)
        b.cgu_scale, b.pam_scale = prm(1, std=0.0, mean=1.0)[0], prm(1, std=0.0, mean=0.1)[0]
        b.pam = _BenchPamLayer(dim, H, d, M, 16, torch.float32, seed=40 + i).mod
        blocks.append(b)
    model.blocks = blocks
    return model


def bench_model_decode(steps, warmup, dtype="bf16", graphs=True):
    """Model-level continuous-batching decode (qllm2_amd.model_decode.ModelDecoder):
    the whole V11 model per token for the live rows of 256 slots (~75% live):
    embedding, 16 blocks (ComplexNorm -> CGU with ModSwish, hidden 3 * 768 ->
    ComplexNorm -> E3 PAM layer M=3, H=12, d=64) and the tied LM head over the
    50261-entry vocabulary (logits of every live row).  GEMMs in `dtype` (fp32
    accumulation; states, norms and the decode kernel in fp32); with `graphs`
    each live-count bucket of 16 rows is captured once and replayed."""
    import torch
    from qllm2_amd.model_decode import ModelDecoder
    S, L, H, d, M, dim, V = 256, 16, 12, 64, 3, 768, 50261
    model = _bench_model(L, dim, H, d, M, V, 3)
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dec = ModelDecoder(model, n_slots=S, max_len=8192, dtype=dt, graphs=graphs, graph_bucket=16)
    if graphs:
        warmup = max(warmup, 16)
    gen = torch.Generator().manual_seed(1017)
    for s_ in range(S):
        dec.engine.admit(int(torch.randint(1, 4096, (1,), generator=gen)))
    dec.pool.state.normal_(0.0, 0.01, generator=torch.Generator(device="cuda").manual_seed(1018))
    hosts = [torch.nonzero(torch.rand(S, generator=gen) < 0.75).flatten().tolist() for _ in range(16)]
    masks = [torch.tensor(h, dtype=torch.int32).cuda() for h in hosts]
    ids = [torch.randint(0, V, (len(h),), generator=gen).cuda() for h in hosts]

    def step(i):
        dec.step(ids[i % 16], masks[i % 16], host_slots=hosts[i % 16])

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    active = sum(len(hosts[i % 16]) for i in range(steps)) / steps
    return {"config": f"V11 model decode: 16 blocks (CGU expand 3, E3 PAM M=3, H=12, d=64), dim=768, vocab {V}, "
                      f"{dtype} GEMMs, 256 slots (~75% live)" + (", HIP-graph replay per bucket of 16" if graphs else ""),
            "ms_per_step": ms, "tokens_per_s": active / (ms * 1e-3), "active_slots": active, "steps": steps}


def bench_e3_fwd_bwd(steps, warmup):
    """Config 3: E3 M=3 scan forward + backward, bf16 q/k/v, fp32 state."""
    import torch
    from qllm2_amd.pam_scan import pam_scan_planar
    from oracle.pam import scan_flops
    M, B, H, T, d, C = 3, 8, 12, 2048, 64, 64
    (qr, qi), (kr, ki), (vr, vi), gamma = scan_inputs(B, H, T, d, M, 1003, torch.bfloat16, mu=2.0, mu_step=1.0)
    leaves = [x.requires_grad_(True) for x in (qr, qi, kr, ki, vr, vi, gamma)]
    gen = torch.Generator().manual_seed(1004)
    dy = torch.randn(B, H, T, d, 2, generator=gen)
    dy_re, dy_im = dy[..., 0].contiguous().cuda(), dy[..., 1].contiguous().cuda()

    def step():
        y_re, y_im, _, _ = pam_scan_planar(*leaves, q_scale=d ** -0.5, chunk=C)
        torch.autograd.backward([y_re, y_im], [dy_re, dy_im])
        for x in leaves:
            x.grad = None

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = scan_flops(B, H, T, d, C, M, backward=True)
    return {"ms_per_step": ms, "tokens_per_s": B * T / (ms * 1e-3), "tflops": flops / (ms * 1e-3) / 1e12,
            "bf16_mfma_frac": flops / (ms * 1e-3) / MFMA_BF16_PEAK, "flops": flops,
            "config": "M=3 B=8 T=2048 H=12 d=64 C=64 bf16 in, fp32 state, fwd+bwd"}


def bench_ce(steps, warmup, master_fp32=False):
    """Config 5: tied complex LM-head CE fwd+bwd, N=16384, D=1024, V=50261, bf16
    (master_fp32: an fp32 master E, run on its bf16 copy, fp32 dE)."""
    import torch
    from qllm2_amd.fused_ce import fused_linear_cross_entropy
    from oracle.ce import ce_flops, make_ce_inputs
    N, d_model, V = 16384, 512, 50261
    h, w, t = make_ce_inputs(N, d_model, V, 1005, dtype=torch.bfloat16)
    if master_fp32:
        w = w.float()
    h, w, t = h.cuda().requires_grad_(True), w.cuda().requires_grad_(True), t.cuda()

    def step():
        loss = fused_linear_cross_entropy(h, w, t)
        loss.backward()
        h.grad = None
        w.grad = None

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = ce_flops(N, V, 2 * d_model)
    return {"ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3), "tflops": flops / (ms * 1e-3) / 1e12,
            "bf16_mfma_frac": flops / (ms * 1e-3) / MFMA_BF16_PEAK, "flops": flops,
            "config": "N=16384 D=1024 V=50261 bf16" + (", fp32 master E" if master_fp32 else "") + ", chunk=4096, fwd+bwd"}


def bench_complex_ops(steps, warmup):
    """Complex elementwise layers (ComplexNorm, ModSwish, CGU gate), forward +
    backward, on [65536, 1024] complex bf16 rows (4 batches of 16k tokens at dim
    1024: large enough that the kernels, not the Python launches, set the
    time).  HBM-bound: algorithmic bytes per call are the complex tensors read
    and written (2 bytes per real), parameters aside."""
    import torch
    from qllm2_amd import triton_kernels as tk
    rows, dim = 65536, 1024
    g = torch.Generator(device="cuda").manual_seed(9)
    z = torch.randn(rows, dim, 2, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    up = torch.randn(rows, dim, 2, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    gout = torch.randn(rows, dim, 2, device="cuda", generator=g).to(torch.bfloat16)
    scale = torch.ones(dim, device="cuda", requires_grad=True)
    bias = torch.zeros(dim, device="cuda", requires_grad=True)
    beta = torch.ones(dim, device="cuda", requires_grad=True)
    el = rows * dim * 2 * 2  # bytes of one complex bf16 tensor
    cases = {
        # forward reads z (+ up), writes out; backward reads z (+ up) and gout, writes gz (+ gup)
        "complex_norm": (lambda: tk.fused_complex_norm(z, scale), (z, scale), 2 * el + 3 * el),
        "mod_swish": (lambda: tk.fused_mod_swish(z, bias, beta), (z, bias, beta), 2 * el + 3 * el),
        "cgu_gate": (lambda: tk.fused_cgu_gate(z, up), (z, up), 3 * el + 5 * el),
    }
    res = {}
    for name, (fn, inputs, nbytes) in cases.items():
        def step():
            torch.autograd.grad(fn(), inputs, gout)  # no .grad accumulation in the timed loop
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        res[name] = {"ms_fwd_bwd": ms, "GBps": nbytes / (ms * 1e-3) / 1e9,
                     "hbm_frac": nbytes / (ms * 1e-3) / HBM_PEAK, "bytes": nbytes}
    res["config"] = "rows=65536 dim=1024 complex bf16, fwd+bwd"
    return res


class _BenchPamLayer:
    """Parameters and attributes of a V11PAMLayer in the production E3 setting
    (fused QKV, RoPE, GSP gate on |x|, K phase-routed states, head decay,
    additive write), random-initialised, for timing the layer forward+backward
    two ways: the fused path (qllm2_amd.pam_layer.forward) and the reference's
    sequence of elementwise torch steps around the same scan kernels."""

    def __init__(self, dim, H, d, M, T, dtype, seed=21):
        import torch
        from qllm2_amd.decode import build_rope_cache
        g = torch.Generator().manual_seed(seed)
        inner = H * d

        def prm(*shape, std):
            return torch.nn.Parameter((torch.randn(*shape, generator=g) * std).to("cuda", dtype))

        mod = torch.nn.Module()
        mod.num_heads, mod.head_dim, mod.n_states, mod.inner_dim = H, d, M, inner
        mod.chunk_size, mod.use_rope, mod.use_gsp, mod.qk_norm, mod.fused_qkv = 256, True, True, False, True
        mod.gamma_floor, mod.gate_content_aware, mod.routing_content_aware, mod.state_compete = 0.0, False, False, False
        mod.decay_mode, mod.write_mode, mod.fused_e3, mod.gate_surprisal_lambda = "head", "additive", True, 0.0
        for name, o, i in (("qkv_proj", 3 * inner, dim), ("o_proj", dim, inner)):
            lin = torch.nn.Module()
            lin.weight_real, lin.weight_imag, lin.bias_real = prm(o, i, std=i ** -0.5), prm(o, i, std=i ** -0.5), None
            setattr(mod, name, lin)
        mod.dt_proj = torch.nn.Linear(2 * dim, H).to("cuda", dtype)
        mod.dt_bias = prm(H, std=0.5)
        mod.protect_gate = torch.nn.Linear(dim, H).to("cuda", dtype)
        mod.state_dt_offset = prm(M, std=1.0)
        mod.phase_proj = torch.nn.Linear(dim, H * M).to("cuda", dtype)
        mod.register_buffer("rope_cache", build_rope_cache(2 * T, d, device="cuda"), persistent=False)
        mod.dropout = torch.nn.Dropout(0.0)
        mod.training = False

        def phase_and_alpha(x):
            b, t = x.shape[:2]
            phase = mod.phase_proj(torch.sqrt(x[..., 0].square() + x[..., 1].square() + 1e-8)).view(b, t, H, M)
            return phase, torch.ones_like(phase)
        mod._phase_and_alpha = phase_and_alpha
        mod._route_balance_loss = lambda w: None
        self.mod = mod

    def fused(self, x):
        from qllm2_amd import pam_layer
        return pam_layer.forward(self.mod, x, None, 0)

    def unfused(self, x):
        """The reference's forward steps (v11/model.py:271-306, 630-655,
        739-781, 834-836) as separate torch passes, the scan itself on the
        same HIP kernels."""
        import torch
        import torch.nn.functional as F
        from qllm2_amd.pam_scan import pam_scan_interleaved
        m = self.mod
        b, t = x.shape[:2]
        H, d, M = m.num_heads, m.head_dim, m.n_states

        def clin(lin, z):
            re = F.linear(z[..., 0], lin.weight_real) - F.linear(z[..., 1], lin.weight_imag)
            im = F.linear(z[..., 0], lin.weight_imag) + F.linear(z[..., 1], lin.weight_real)
            return torch.stack([re, im], -1)

        def cmul(a, r):
            return torch.stack([a[..., 0] * r[..., 0] - a[..., 1] * r[..., 1],
                                a[..., 0] * r[..., 1] + a[..., 1] * r[..., 0]], -1)

        qkv = clin(m.qkv_proj, x).view(b, t, 3, H, d, 2)
        q, k, v = (qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3))
        rope = m.rope_cache[:t].to(x.dtype)
        q, k = cmul(q, rope), cmul(k, rope)
        phase, routing = m._phase_and_alpha(x)
        phase, routing = phase.permute(3, 0, 2, 1), routing.permute(3, 0, 2, 1)
        x_flat = torch.cat([x[..., 0], x[..., 1]], -1)
        sp = F.softplus(m.dt_proj(x_flat) + m.dt_bias + m.state_dt_offset.view(M, 1, 1, 1))
        base = torch.exp(-sp.permute(0, 1, 3, 2).contiguous())
        p = torch.sigmoid(m.protect_gate(torch.sqrt(x[..., 0].square() + x[..., 1].square() + 1e-8))).transpose(1, 2)
        gamma = base * (1 - p) + p
        v = v * (1 - p)[..., None, None]
        rot = (routing * torch.cos(phase), routing * torch.sin(phase))
        y, s = pam_scan_interleaved(q, k, v, gamma, d, m.chunk_size, rot=rot)
        y = y.transpose(1, 2).contiguous().view(b, t, H * d, 2)
        return clin(m.o_proj, y), s


def bench_pam_layer(steps, warmup):
    """PAM layer forward + backward at the config-3 shape (E3 M=3, B=8, T=2048,
    H=12, d=64, dim=768, bf16 parameters and activations): the fused path
    against the reference's unfused elementwise steps around the same scan,
    and the prologue kernels alone (HBM-bound: algorithmic bytes are the six
    projection planes read and the six scan operand planes written, plus the
    per-token scalars)."""
    import torch
    from qllm2_amd import pam_prologue as PP
    B, T, H, d, M, dim = 8, 2048, 12, 64, 3, 768
    lay = _BenchPamLayer(dim, H, d, M, T, torch.bfloat16)
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(B, T, dim, 2, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    dy = torch.randn(B, T, dim, 2, device="cuda", generator=g).to(torch.bfloat16)
    params = [p for p in lay.mod.parameters()]
    res = {"config": "E3 M=3, B=8, T=2048, H=12, d=64, dim=768, bf16, fwd+bwd"}
    for name, fn in (("fused", lay.fused), ("unfused_reference_steps", lay.unfused)):
        def step():
            out, _ = fn(x)
            torch.autograd.grad(out, [x] + params, dy)
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        res[name + "_ms"] = e0.elapsed_time(e1) / steps
    res["speedup"] = res["unfused_reference_steps_ms"] / res["fused_ms"]
    # the prologue kernels alone, fed the layer's own tensors
    from qllm2_amd import pam_layer as PL
    m = lay.mod
    with torch.no_grad():
        cols = PP.proj_columns(H, d)
        w_in, b_in = PL._in_weight(m, H, d, cols)
        proj = torch.nn.functional.linear(x.detach().view(B, T, 2 * dim), w_in, b_in)
        mag = torch.sqrt(x.detach().square().sum(-1) + 1e-8)
        prot = m.protect_gate(mag)
        phase = m.phase_proj(mag).view(B, T, H, M)
    args = (proj, prot, phase, None, m.dt_bias.detach().float(), None, m.state_dt_offset.detach().float(),
            m.rope_cache, H, M, d, 0, False, 0.0, None, -1, -1)
    outs = PP.prologue_fwd_op(*args)
    grads = [torch.randn_like(o) if o.numel() else o for o in outs]
    plane = B * T * H * d * 2                  # bytes of one bf16 plane
    tok = B * T * H * 4                        # one fp32 value per (token, head)
    tok2 = B * T * H * 2                       # one bf16 value per (token, head)
    # forward: 6 projection planes in, 6 operand planes out; dt, protect, M phases in (bf16); gamma, rot out (fp32)
    fwd_bytes = 12 * plane + (2 + M) * tok2 + 3 * M * tok
    # backward: 6 gradient planes and the 2 v planes in, 6 projection-gradient planes out; the logits in again;
    # dgamma, drot in; dphase, dprotect, ddt out (bf16); the bias gradients as per-block partial sums
    bwd_bytes = 14 * plane + (2 + M) * tok2 + 3 * M * tok + (M + 2) * tok2
    for name, fn, nbytes in (("prologue_fwd", lambda: PP.prologue_fwd_op(*args), fwd_bytes),
                             ("prologue_bwd", lambda: PP.prologue_bwd_op(*args, grads), bwd_bytes)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 20
        res[name] = {"ms": ms, "bytes": nbytes, "GBps": nbytes / (ms * 1e-3) / 1e9,
                     "hbm_frac": nbytes / (ms * 1e-3) / HBM_PEAK}
    return res


def _delta_reference_steps(q, k, v, gamma, beta, d, chunk):
    """The reference's chunked E2 forward (v11/model.py:491-576) as torch
    steps on the GPU -- decay matrix, Gram and mass matrices, the 2C x 2C real
    block solve, dual-form and carried reads, state write -- for timing
    against the kernels.  Planar fp32 inputs [B,H,T,d]."""
    import torch
    (qr, qi), (kr, ki), (vr, vi) = q, k, v
    B, H, T, _ = qr.shape
    scale = d ** -0.5
    sr = qr.new_zeros(B, H, d, d)
    si = qr.new_zeros(B, H, d, d)
    ys = []
    for c0 in range(0, T, chunk):
        c1 = min(c0 + chunk, T)
        n = c1 - c0
        g, bt = gamma[:, :, c0:c1], beta[:, :, c0:c1]
        lg = torch.log(g + 1e-6)
        cum = torch.cumsum(lg, -1)
        diff = cum.unsqueeze(-1) - cum.unsqueeze(-2)
        dmat = torch.exp(torch.clamp(diff.masked_fill(torch.ones(n, n, device=g.device).triu(1).bool(), -1e4),
                                     max=0)) * torch.ones(n, n, device=g.device).tril()
        alpha = torch.exp(cum)
        k_r, k_i, q_r, q_i = kr[:, :, c0:c1], ki[:, :, c0:c1], qr[:, :, c0:c1], qi[:, :, c0:c1]
        gram_r = k_r @ k_r.transpose(-1, -2) + k_i @ k_i.transpose(-1, -2)
        gram_i = k_i @ k_r.transpose(-1, -2) - k_r @ k_i.transpose(-1, -2)
        strict = torch.ones(n, n, device=g.device).tril(-1)
        m_r, m_i = bt.unsqueeze(-1) * dmat * strict * gram_r, bt.unsqueeze(-1) * dmat * strict * gram_i
        sk_r = (k_r @ sr.transpose(-1, -2) - k_i @ si.transpose(-1, -2)) * alpha.unsqueeze(-1)
        sk_i = (k_r @ si.transpose(-1, -2) + k_i @ sr.transpose(-1, -2)) * alpha.unsqueeze(-1)
        w_r, w_i = bt.unsqueeze(-1) * (vr[:, :, c0:c1] - sk_r), bt.unsqueeze(-1) * (vi[:, :, c0:c1] - sk_i)
        eye = torch.eye(n, device=g.device)
        sysm = torch.cat([torch.cat([eye + m_r, -m_i], -1), torch.cat([m_i, eye + m_r], -1)], -2)
        sol = torch.linalg.solve(sysm, torch.cat([w_r, w_i], -2))
        u_r, u_i = sol[..., :n, :], sol[..., n:, :]
        qk_r = q_r @ k_r.transpose(-1, -2) + q_i @ k_i.transpose(-1, -2)
        qk_i = q_i @ k_r.transpose(-1, -2) - q_r @ k_i.transpose(-1, -2)
        p_r, p_i = dmat * qk_r, dmat * qk_i
        sq_r, sq_i = q_r * scale * alpha.unsqueeze(-1), q_i * scale * alpha.unsqueeze(-1)
        y_r = (p_r @ u_r - p_i @ u_i) * scale + sq_r @ sr.transpose(-1, -2) - sq_i @ si.transpose(-1, -2)
        y_i = (p_r @ u_i + p_i @ u_r) * scale + sq_r @ si.transpose(-1, -2) + sq_i @ sr.transpose(-1, -2)
        ys.append(torch.stack([y_r, y_i], -1))
        tail = (alpha[:, :, -1:] / (alpha + 1e-12)).unsqueeze(-1)
        ud_r, ud_i = u_r * tail, u_i * tail
        total = alpha[:, :, -1:].unsqueeze(-1)
        sr, si = (sr * total + ud_r.transpose(-1, -2) @ k_r + ud_i.transpose(-1, -2) @ k_i,
                  si * total + ud_i.transpose(-1, -2) @ k_r - ud_r.transpose(-1, -2) @ k_i)
    return torch.cat(ys, 2), (sr, si)


def bench_delta(steps, warmup, reference=True):
    """E2 delta rule forward + backward at the config-3 shape (one state: B=8,
    T=2048, H=12, d=64, fp32): the HIP kernels against the reference's chunked
    UT-transform steps (delta_chunk 64) run in torch on the same GPU.  The
    kernels walk the chunks of each (b, h) chain in sequence (forward, and the
    backward's state-gradient pass): `us_per_token` is the forward's time per
    token step; achieved HBM traffic (inputs, outputs, the backward's
    per-chunk records) is reported beside it."""
    import torch
    from qllm2_amd.pam_delta import delta_planar
    B, H, T, d = 8, 12, 2048, 64
    gen = torch.Generator(device="cuda").manual_seed(31)
    planes = [torch.randn(B, H, T, d, device="cuda", generator=gen) for _ in range(6)]
    nrm = (planes[2].square() + planes[3].square()).sum(-1, keepdim=True).sqrt()
    planes[2], planes[3] = planes[2] / nrm, planes[3] / nrm
    gamma = 0.5 + 0.5 * torch.sigmoid(torch.randn(B, H, T, device="cuda", generator=gen) + 2)
    beta = torch.sigmoid(torch.randn(B, H, T, device="cuda", generator=gen))
    leaves = [x.requires_grad_(True) for x in planes + [gamma, beta]]
    dy = [torch.randn(B, H, T, d, device="cuda", generator=gen) for _ in range(2)]

    def timed(fn, n):
        for _ in range(min(warmup, n)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    def fused():
        y_re, y_im, _, _ = delta_planar(*leaves[:6], leaves[6], leaves[7], q_scale=d ** -0.5)
        torch.autograd.grad([y_re, y_im], leaves, dy)

    def fwd_only():
        with torch.no_grad():
            delta_planar(*planes, gamma, beta, q_scale=d ** -0.5)

    def reference_steps():
        y, _ = _delta_reference_steps((leaves[0], leaves[1]), (leaves[2], leaves[3]), (leaves[4], leaves[5]),
                                      leaves[6], leaves[7], d, 64)
        torch.autograd.grad([y[..., 0], y[..., 1]], leaves, dy)

    if reference == "only":  # the torch reference steps alone (never under a counter pass)
        ref_ms = timed(reference_steps, max(2, steps // 5))
        return {"config": "E2 reference steps, B=8 T=2048 H=12 d=64 fp32, fwd+bwd", "ms_fwd_bwd": ref_ms}
    ms = timed(fused, steps)
    fwd_ms = timed(fwd_only, steps)
    fwd_bytes = 6 * B * H * T * d * 4 + 2 * B * H * T * 4 + 2 * B * H * T * d * 4 + B * H * (T // 16) * 2 * d * d * 4
    out = {"config": "E2 delta write, B=8 T=2048 H=12 d=64 fp32, fwd+bwd", "ms_fwd_bwd": ms, "ms_fwd": fwd_ms,
           "tokens_per_s": B * T / (ms * 1e-3), "us_per_token_fwd": fwd_ms * 1e3 / T, "fwd_bytes": fwd_bytes,
           "fwd_hbm_frac": fwd_bytes / (fwd_ms * 1e-3) / HBM_PEAK}
    if reference:
        out["reference_steps_ms_fwd_bwd"] = timed(reference_steps, max(2, steps // 5))
        out["speedup"] = out["reference_steps_ms_fwd_bwd"] / ms
    return out


def _perchannel_reference_steps(q, k, v, gamma, d, chunk):
    """The reference's E1 chunked prefill (v11/model.py:421-489) as torch steps
    on the GPU, for timing against the kernels: per chunk the decay fold, the
    masked score, its read of V, the carried read and the state write.
    Interleaved complex inputs [B,H,T,d,2], gamma [B,H,T,d]."""
    import torch
    B, H, T = q.shape[:3]
    scale = d ** -0.5
    st = q.new_zeros(B, H, d, d, 2)
    outs = []
    for c0 in range(0, T, chunk):
        c1 = min(c0 + chunk, T)
        n = c1 - c0
        lg = torch.cumsum(torch.log(gamma[:, :, c0:c1].clamp_min(1e-6)), 2).clamp(min=-30.0)
        a, inv, tail = torch.exp(lg), torch.exp(-lg), torch.exp(lg[:, :, -1:] - lg)
        fq, fk = q[:, :, c0:c1] * (a * scale).unsqueeze(-1), k[:, :, c0:c1] * inv.unsqueeze(-1)
        wr = fq[..., 0] @ fk[..., 0].transpose(-1, -2) + fq[..., 1] @ fk[..., 1].transpose(-1, -2)
        wi = fq[..., 1] @ fk[..., 0].transpose(-1, -2) - fq[..., 0] @ fk[..., 1].transpose(-1, -2)
        mask = torch.ones(n, n, device=q.device).tril()
        wr, wi = wr * mask, wi * mask
        vr, vi = v[:, :, c0:c1, :, 0], v[:, :, c0:c1, :, 1]
        o_r, o_i = wr @ vr - wi @ vi, wr @ vi + wi @ vr
        if c0 > 0:
            sr, si = st[..., 0], st[..., 1]
            o_r = o_r + fq[..., 0] @ sr.transpose(-1, -2) - fq[..., 1] @ si.transpose(-1, -2)
            o_i = o_i + fq[..., 0] @ si.transpose(-1, -2) + fq[..., 1] @ sr.transpose(-1, -2)
        outs.append(torch.stack([o_r, o_i], -1))
        dk = k[:, :, c0:c1] * tail.unsqueeze(-1)
        s_r = vr.transpose(-1, -2) @ dk[..., 0] + vi.transpose(-1, -2) @ dk[..., 1]
        s_i = vi.transpose(-1, -2) @ dk[..., 0] - vr.transpose(-1, -2) @ dk[..., 1]
        st = st * torch.exp(lg[:, :, -1])[:, :, None, :, None] + torch.stack([s_r, s_i], -1)
    return torch.cat(outs, 2), st


def bench_perchannel(steps, warmup, reference=True):
    """E1 per-channel decay prefill forward + backward at the config-3 shape
    (one state: B=8, T=2048, H=12, d=64, chunk 64, fp32): the HIP fold and
    state-scan kernels around batched complex GEMMs against the reference's
    per-chunk steps run in torch on the same GPU."""
    import torch
    from qllm2_amd.pam_perchannel import perchannel_chunked
    B, H, T, d = 8, 12, 2048, 64
    gen = torch.Generator(device="cuda").manual_seed(41)
    q, k, v = (torch.randn(B, H, T, d, 2, device="cuda", generator=gen) * (2 * d) ** -0.5 for _ in range(3))
    gamma = torch.sigmoid(torch.randn(B, H, T, d, device="cuda", generator=gen) + 3.0)
    leaves = [x.requires_grad_(True) for x in (q, k, v, gamma)]
    dy = torch.randn(B, H, T, d, 2, device="cuda", generator=gen)

    def timed(fn, n):
        for _ in range(min(warmup, n)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    def fused():
        y, _ = perchannel_chunked(*leaves, d, 64)
        torch.autograd.grad([y], leaves, [dy])

    def fwd_only():
        with torch.no_grad():
            perchannel_chunked(q, k, v, gamma, d, 64)

    def reference_steps():
        y, _ = _perchannel_reference_steps(*leaves, d, 64)
        torch.autograd.grad([y], leaves, [dy])

    ms = timed(fused, steps)
    out = {"config": "E1 per-channel decay, B=8 T=2048 H=12 d=64 chunk 64 fp32, fwd+bwd", "ms_fwd_bwd": ms,
           "ms_fwd": timed(fwd_only, steps), "tokens_per_s": B * T / (ms * 1e-3)}
    if reference:
        out["reference_steps_ms_fwd_bwd"] = timed(reference_steps, max(2, steps // 5))
        out["speedup"] = out["reference_steps_ms_fwd_bwd"] / ms
    return out


def _median_time(fn, reps):
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline_scan():
    """The reference's chunk loop restated on the CPU (oracle.pam.chunked_head),
    fp32, on a bounded sample: 1 of the 8 batch rows (H=12, T=2048)."""
    import torch
    from oracle.pam import chunked_head, make_scan_inputs
    threads = cpu_threads()
    torch.set_num_threads(threads)
    q, k, v, gamma = make_scan_inputs(1, 12, 2048, 64, 1002, unit_qk=True, dtype=torch.float32)
    chunked_head(q, k, v, gamma[0], 64, 64)
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        chunked_head(q, k, v, gamma[0], 64, 64)
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    out = {"value": 2048 / t, "unit": "tokens/s", "cores": threads, "kind": "port",
           "sample": "oracle.pam.chunked_head fp32, B=1 of 8 (H=12, T=2048, d=64, C=64), median of 3"}
    out.update(host_info(threads))
    return out


def cpu_baseline_e3():
    """Config 3 on the CPU: the reference's fused E3 chunk loop restated in torch
    (oracle.pam.multistate_fused, v11/model.py:657-781), fp32 forward plus
    autograd backward on the bf16-rounded inputs, 1 of the 8 batch rows."""
    import torch
    from oracle import pam as O
    threads = cpu_threads()
    torch.set_num_threads(threads)
    M, B, H, T, d, C = 3, 1, 12, 2048, 64, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 1003, m_states=M, gamma_mu=2.0, gamma_mu_step=1.0,
                                        unit_qk=True, dtype=torch.float32)
    q, k, v = (x.to(torch.bfloat16).to(torch.float32) for x in (q, k, v))
    dy = torch.randn(B, H, T, d, 2, generator=torch.Generator().manual_seed(1004))
    phase, routing = torch.zeros(M, B, H, T), torch.ones(M, B, H, T)

    def step():
        xs = [x.clone().requires_grad_(True) for x in (q, k, v, gamma)]
        y, _ = O.multistate_fused(xs[0], xs[1], xs[2], xs[3], phase, routing, d, C)
        (y * dy).sum().backward()

    t = _median_time(step, 3)
    out = {"value": B * T / t, "unit": "tokens/s", "kind": "port",
           "sample": "oracle.pam.multistate_fused fp32 forward + autograd backward, M=3, B=1 of 8 "
                     "(H=12, T=2048, d=64, C=64), median of 3"}
    out.update(host_info(threads))
    return out


def cpu_baseline_decode(steps=20):
    """Config 4 on the CPU: the reference's token step (oracle.pam.recur_step_additive,
    v11/model.py:927-965) over 16 layers x 12 heads for a sample of 16 live
    slots, `steps` consecutive tokens, fp32."""
    import torch
    from oracle import pam as O
    threads = cpu_threads()
    torch.set_num_threads(threads)
    S, G, d = 16, 16 * 12, 64
    gen = torch.Generator().manual_seed(1004)
    state = torch.randn(S, G, d, d, 2, generator=gen) * 0.01
    gamma = torch.sigmoid(torch.randn(S, G, generator=gen) + 3)
    qkv = [torch.randn(3, S, G, d, 2, generator=gen) for _ in range(steps)]
    O.recur_step_additive(state, gamma, qkv[0][2], qkv[0][1], qkv[0][0] * d ** -0.5)
    t0 = time.perf_counter()
    for x in qkv:
        _, state = O.recur_step_additive(state, gamma, x[2], x[1], x[0] * d ** -0.5)
    t = time.perf_counter() - t0
    out = {"value": S * steps / t, "unit": "tokens/s", "kind": "port",
           "sample": f"oracle.pam.recur_step_additive fp32, 16 live slots x 16 layers x 12 heads (d=64), "
                     f"{steps} consecutive steps"}
    out.update(host_info(threads))
    return out


def cpu_baseline_ce():
    """Config 5 on the CPU: the reference's chunked fused CE restated in torch
    (oracle.ce ce_forward / ce_backward, v11/fused_ce.py:28-82), fp32 on the
    bf16-rounded inputs, 512 of the 16384 rows against the full vocabulary."""
    import torch
    from oracle.ce import ce_backward, ce_forward, make_ce_inputs
    threads = cpu_threads()
    torch.set_num_threads(threads)
    N, d_model, V = 512, 512, 50261
    h, w, tgt = make_ce_inputs(N, d_model, V, 1005, dtype=torch.bfloat16)
    h, w = h.float(), w.float()

    def step():
        _, denom = ce_forward(h, w, tgt, chunk=N)
        ce_backward(h, w, tgt, denom, chunk=N)

    t = _median_time(step, 3)
    out = {"value": N / t, "unit": "tokens/s", "kind": "port",
           "sample": "oracle.ce ce_forward + ce_backward fp32, 512 of 16384 rows, V=50261, D=1024, median of 3"}
    out.update(host_info(threads))
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    if args.only is not None:
        fn = {"scan_fwd": lambda: dict(zip(("ms", "kernel_ms", "tokens", "flops", "kernel_flops", "kernel_flops_causal"),
                                           bench_scan_fwd(args.steps, args.warmup))),
              "decode": lambda: bench_decode(args.decode_steps),
              "decode_e3": lambda: bench_decode_e3_rope(max(50, args.decode_steps // 5)),
              "engine": lambda: {"eager": bench_engine(args.steps, args.warmup),
                                 "graphs": bench_engine(args.steps, args.warmup, graphs=True),
                                 "graphs_bf16": bench_engine(args.steps, args.warmup, graphs=True, dtype="bf16")},
              "model": lambda: {"bf16_graphs": bench_model_decode(args.steps, args.warmup),
                                "fp32_graphs": bench_model_decode(args.steps, args.warmup, dtype="fp32"),
                                "bf16_eager": bench_model_decode(args.steps, args.warmup, graphs=False)},
              "e3": lambda: bench_e3_fwd_bwd(args.steps, args.warmup),
              "ce": lambda: bench_ce(args.steps, args.warmup),
              "cplx": lambda: bench_complex_ops(args.steps, args.warmup),
              "layer": lambda: bench_pam_layer(args.steps, args.warmup),
              "delta": lambda: bench_delta(args.steps, args.warmup, reference=False),
              "delta_ref": lambda: bench_delta(args.steps, args.warmup, reference="only"),
              "e1": lambda: bench_perchannel(args.steps, args.warmup),
              "copy": copy_calibration}[args.only]
        print(json.dumps({"only": args.only, "result": fn()}), flush=True)
        return
    ms, kms, tokens, flops, kflops, kflops_causal = bench_scan_fwd(args.steps, args.warmup)
    value = tokens / (ms * 1e-3)
    achieved = kflops / (kms * 1e-3)
    traffic, traffic_build = measured_traffic("scan_fwd/chunk_output_f32_kernel<64>")
    out = {
        "metric": "PAM prefill tokens/s + MFMA %; ragged decode tokens/s + HBM GB/s (256 slots)",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded CPU draws, BASELINE.json config 2)",
        "config": {"workload": "config 2: PAM chunked dual-form scan forward (prefill), fp32 complex",
                   "B": 8, "T": 2048, "H": 12, "d": 64, "C": 64,
                   "layout": "planar re/im fp32"},
        "roofline": {"bound": "mfma", "achieved": achieved / 1e12, "peak": MFMA_FP32_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": achieved / MFMA_FP32_PEAK,
                     "frac_causal": kflops_causal / (kms * 1e-3) / MFMA_FP32_PEAK,
                     "traffic": traffic, "traffic_build": traffic_build, "build": source_hash(),
                     "kernel": "chunk_output_f32_kernel<64>", "kernel_ms": kms,
                     "kernel_flops": kflops, "kernel_flops_causal": kflops_causal},
        "scan_fwd_total": {"flops": flops, "tflops": flops / (ms * 1e-3) / 1e12,
                           "mfma_fp32_frac": flops / (ms * 1e-3) / MFMA_FP32_PEAK},
    }
    if not args.no_extras:
        # the north-star E3 step first, next to the headline scan, with the headline's step count
        out["extras"] = {"e3_fwd_bwd_config3": bench_e3_fwd_bwd(args.steps, max(5, args.warmup)),
                         "decode_config4": bench_decode(args.decode_steps),
                         "decode_e3_rope_slots": bench_decode_e3_rope(max(50, args.decode_steps // 5)),
                         "decode_engine_e3_16_layers": bench_engine(20, 5),
                         "decode_engine_e3_16_layers_graphs": bench_engine(20, 5, graphs=True),
                         "decode_engine_e3_16_layers_graphs_bf16": bench_engine(20, 5, graphs=True, dtype="bf16"),
                         "model_decode_16_blocks_bf16_graphs": bench_model_decode(20, 5),
                         "ce_fwd_bwd_config5": bench_ce(max(3, args.steps // 4), 3),
                         "ce_fwd_bwd_config5_fp32_master_e": bench_ce(max(3, args.steps // 4), 3, master_fp32=True),
                         "complex_elementwise": bench_complex_ops(max(3, args.steps // 2), 5),
                         "pam_layer_config3": bench_pam_layer(max(3, args.steps // 2), 5),
                         "delta_e2_config3_shape": bench_delta(max(3, args.steps // 4), 1),
                         "perchannel_e1_config3_shape": bench_perchannel(max(3, args.steps // 4), 2)}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_scan()
        out["cpu_baselines"] = {"config3_e3_fwd_bwd": cpu_baseline_e3(), "config4_decode": cpu_baseline_decode(),
                                "config5_ce_fwd_bwd": cpu_baseline_ce()}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
