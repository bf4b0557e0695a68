#!/usr/bin/env python3
"""Benchmark of the MI355X PJRT plugin's hot path (one GPU).

Metric: "SDPA TFLOP/s vs seq len (512-16384) & % MFMA peak;
fusion GB/s % HBM peak".

  value      causal SDPA forward, bf16, B=4 H=16 D=128, S=8192 (config C3 at
             the north_star target length), TFLOP/s with FLOPs = 2*B*H*S^2*D
             (causal half of 4*B*H*S^2*D).  One step = one mk_sdpa_fwd launch
             over inputs already resident in HBM.
  sweep      the same for S in 512..16384
  fusions    C2 LayerNorm / GELU / reduce_sum / argmax and C4 gather /
             scatter-add, GB/s of algorithmic bytes and fraction of 8 TB/s
  roofline   the dominant kernel (SDPA at S=8192): achieved TFLOP/s from HIP
             events on the launch stream, against 2516.6 TFLOP/s bf16 dense
  cpu_baseline  an fp32 torch-CPU restatement (not XLA:CPU; jax is absent)
             on a bounded sample of (b, h) pairs of the same workload, scaled
             to all pairs, with the thread count
  cpu_baselines_other_configs  the same kind of restatement for C1, the C2 and
             C4 fusions and the C5 training step (bounded samples, in each
             GPU figure's unit)
  gemm       the C5 step's 15 GEMM shapes on mk_gemm and rocBLAS, and C1
             through PJRT Execute (TFLOP/s, fraction of the fp32 peak)
  pjrt_execute  the same attention through PJRT_LoadedExecutable_Execute
             (the plugin path), and the per-Execute cost of a tiny module
  training_step  config C5: one GPT-2-small training step (forward, backward,
             Adam; 12 layers, d 768, 12 heads, seq 1024, batch 8, vocab
             50257, bf16 activations, fp32 Adam) replayed as one HIP graph;
             ms/step, tokens/s, model TFLOP/s (3x forward FLOPs) and MFU

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--spinup SECONDS]
       [--only sdpa|fusions|headline|calib|c5|gemm|pjrt]

Before the first timed region the headline kernel runs untimed for --spinup
seconds (default 1), so that no timed region includes the clocks' ramp from
idle; then each workload runs W untimed and K timed launches.  Each SDPA
sequence length first runs untimed on its own inputs (--spinup seconds at the
headline length, up to 0.2 s at the others): the host-side input generation
before it leaves the GPU idle long enough for the clocks to drop, and after
that the first ~50 ms of launches run up to 10% slower than the sustained
rate, which 10 warm-up launches do not cover.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "mccl-jax_amd"))

PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--spinup", type=float, default=1.0,
                    help="seconds of untimed headline launches before anything is timed (clocks settle)")
    ap.add_argument("--only", choices=["sdpa", "fusions", "headline", "calib", "c5", "gemm", "pjrt", "c5jit", "c1"], default=None)
    ap.add_argument("--seq", type=int, default=8192, help="headline sequence length")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    return ap.parse_args()


def dev_bf16(bits, torch, np):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def time_launches(torch, fn, steps, warmup):
    """Average milliseconds per call of fn (one or more launches on torch's
    current stream), HIP events around the whole timed region."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def spin_up(torch, np, K, args):
    """Untimed launches of the headline kernel for args.spinup seconds, so that
    the GPU's clocks have left their idle state before the first timed region
    (a cold MI355X runs the first tens of milliseconds of work slower)."""
    if args.spinup <= 0:
        return
    B, H, S, D = 4, 16, 8192, 128
    q = torch.zeros(B, H, S, D, dtype=torch.bfloat16, device="cuda")
    o = torch.empty_like(q)
    t0 = time.time()
    while time.time() - t0 < args.spinup:
        for _ in range(20):
            K.sdpa_fwd(q, q, q, 1 / math.sqrt(D), True, out=o)
        torch.cuda.synchronize()
    del q, o
    torch.cuda.empty_cache()


def spin(torch, fn, seconds):
    """Untimed calls of fn for `seconds`, synchronising every 10 calls."""
    t0 = time.time()
    while time.time() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def sdpa_flops(B, H, S, D):
    return 2.0 * B * H * S * S * D


def read_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary
    (profiles/<name>.txt, line 'traffic_bytes_per_launch: N'), else None."""
    p = os.path.join(ROOT, "profiles", name + ".txt")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_baseline_sdpa(torch, np, S, budget_s, gpu_out=None):
    """CPU baseline: an fp32 torch-CPU restatement of the jitted computation
    (einsum -> scale -> where(tril) -> softmax -> einsum, as BASELINE.md's
    fallback plan specifies when jax is absent; it is NOT XLA:CPU) on (b, h)
    pairs of the C3 workload until the time budget is used, then scaled to
    all B*H = 64 pairs.  torch uses every core of this process's affinity
    mask.  The first pair is compared with the GPU result (gpu_out)."""
    from oracle import bf16, inputs

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    d = inputs.c3_sdpa(S)
    B, H, D = 4, 16, 128
    scale = 1 / math.sqrt(D)
    mask = torch.ones(S, S, dtype=torch.bool).tril_()
    done, err = 0, None
    t0 = time.perf_counter()
    for bh in range(B * H):
        b, h = divmod(bh, H)
        q, k, v = (torch.from_numpy(bf16.from_bf16_bits(d[n][b, h]).astype(np.float32)) for n in ("q", "k", "v"))
        s_ = (q @ k.T) * scale
        s_ = torch.where(mask, s_, torch.tensor(float("-inf")))
        o = torch.softmax(s_, dim=-1) @ v
        if bh == 0 and gpu_out is not None:
            err = float((o - gpu_out[b, h].float().cpu()).abs().max())
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    el = time.perf_counter() - t0
    total_s = el / done * B * H
    return {
        "value": round(sdpa_flops(B, H, S, D) / total_s / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": int(cores),
        "kind": "port",
        "sample": f"CPU restatement, not XLA:CPU: fp32 torch-CPU einsum/where(tril)/softmax/einsum on {done} of "
                  f"{B*H} (b,h) pairs at S={S}, {el:.1f}s, extrapolated x{B*H/done:.1f}; torch threads={cores}"
                  + (f"; max |CPU - GPU| on pair (0,0) = {err:.2e}" if err is not None else ""),
    }


CPU_LABEL = "CPU restatement, not XLA:CPU"


def _cpu_time(fn, budget_s, min_reps=1):
    """Seconds per call of fn on the CPU (at least min_reps calls, until the
    budget is used)."""
    fn()  # first call outside the timing (allocation, thread start)
    n, t0 = 0, time.perf_counter()
    while n < min_reps or time.perf_counter() - t0 < budget_s:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def cpu_baselines(torch, np, budget_s):
    """fp32 torch-CPU restatements of the other configs, each timed on a
    bounded sample for about budget_s seconds and reported in the GPU
    figure's unit (scaled to the full workload where a sample is used).
    Not XLA:CPU (jax is absent); torch runs on every core of this process's
    affinity mask."""
    from oracle import bf16, gpt2_ref, inputs

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    out = {}

    def rec(name, value, unit, sample):
        out[name] = {"value": round(value, 4), "unit": unit, "cores": int(cores), "kind": "port",
                     "sample": f"{CPU_LABEL}: {sample}; torch threads={cores}"}
        log(f"cpu {name}: {value:.3f} {unit}")

    # C1: the MLP forward, full size
    d = inputs.c1_mlp()
    x, w1, b1, w2, b2 = (torch.from_numpy(d[n]) for n in ("x", "w1", "b1", "w2", "b2"))
    sec, n = _cpu_time(lambda: torch.relu(x @ w1 + b1) @ w2 + b2, budget_s, 3)
    rec("c1_mlp_fp32", 2.0 * 256 * 1024 * 4096 * 2 / sec / 1e12, "TFLOP/s",
        f"fp32 x@W1+b1, ReLU, @W2+b2 at full size, {n} calls")
    # C2: bf16 in, fp32 compute, on the first rows; GB/s of the same
    # algorithmic bytes per element as the GPU figures
    rows = 1024
    ln = inputs.c2_layernorm(rows=rows)  # the first rows of the C2 array (same generator stream)
    xl = torch.from_numpy(bf16.from_bf16_bits(ln["x"]))
    gl, bl = (torch.from_numpy(bf16.from_bf16_bits(ln[k])) for k in ("gamma", "beta"))
    sec, n = _cpu_time(lambda: torch.nn.functional.layer_norm(xl, (4096,), gl, bl, 1e-5).to(torch.bfloat16),
                       budget_s / 4)
    rec("layernorm_8192x4096_bf16", rows * 4096 * 4 / sec / 1e9, "GB/s",
        f"torch layer_norm on rows 0..{rows} of [8192,4096] widened to fp32, result to bf16, {n} calls")
    del ln, xl
    xg = torch.from_numpy(bf16.from_bf16_bits(inputs.c2_gelu(rows=256)["x"]))
    sec, n = _cpu_time(lambda: torch.nn.functional.gelu(xg, approximate="tanh").to(torch.bfloat16), budget_s / 4)
    rec("gelu_tanh_8192x16384_bf16", xg.numel() * 4 / sec / 1e9, "GB/s",
        f"torch gelu(tanh) on rows 0..256 of [8192,16384] in fp32, result to bf16, {n} calls")
    del xg
    rows = 8192
    xr = torch.from_numpy(bf16.from_bf16_bits(inputs.c2_reduce(rows=rows)["x"]))
    sec, n = _cpu_time(lambda: xr.sum(dim=1), budget_s / 4)
    rec("reduce_sum_65536x1024_bf16", rows * (1024 * 2 + 4) / sec / 1e9, "GB/s",
        f"fp32 row sums of rows 0..{rows} of [65536,1024], {n} calls")
    sec, n = _cpu_time(lambda: xr.argmax(dim=1), budget_s / 4)
    rec("argmax_65536x1024_bf16", rows * (1024 * 2 + 4) / sec / 1e9, "GB/s",
        f"row argmax of rows 0..{rows} of [65536,1024], {n} calls")
    del xr
    # C4: full size
    c4 = inputs.c4_indexing()
    table = torch.from_numpy(bf16.from_bf16_bits(c4["table_bf16"])).to(torch.bfloat16)
    ids = torch.from_numpy(c4["ids"]).reshape(-1).long()
    sec, n = _cpu_time(lambda: table.index_select(0, ids), budget_s / 2)
    rec("gather_32x2048_from_50257x768_bf16", (65536 * 4 + 2 * 65536 * 768 * 2) / sec / 1e9, "GB/s",
        f"index_select of 65536 rows of [50257,768] bf16, {n} calls")
    tf, gr = torch.from_numpy(c4["table_f32"]), torch.from_numpy(c4["grads"])
    sec, n = _cpu_time(lambda: tf.clone().index_add_(0, ids, gr), budget_s / 2)
    rec("scatter_add_65536x768_into_50257x768_f32", (65536 * 768 * 4 + 65536 * 4 + 2 * 50257 * 768 * 4) / sec / 1e9,
        "GB/s", f"index_add_ of 65536 rows into a copy of [50257,768] fp32, {n} calls")
    del c4, table, tf, gr
    # C5: the GPT-2 step (forward, backward, Adam) for one of the 8 sequences
    from mi355x_pjrt import gpt2

    cfg = gpt2.GPT2Config()
    params = {k: torch.tensor(v, requires_grad=True) for k, v in gpt2.init_params(cfg, 0).items()}
    st = {k: (torch.zeros_like(v), torch.zeros_like(v)) for k, v in params.items()}
    rng = np.random.default_rng(5000)
    ids5 = rng.integers(0, cfg.vocab, (1, cfg.seq)).astype(np.int64)
    labels = np.roll(ids5, -1, axis=1)

    def step():
        loss = gpt2_ref.forward_loss(params, ids5, labels, cfg.n_layer, cfg.n_head)
        loss.backward()
        with torch.no_grad():
            for k, p_ in params.items():
                m, v = st[k]
                m.mul_(0.9).add_(p_.grad, alpha=0.1)
                v.mul_(0.999).addcmul_(p_.grad, p_.grad, value=0.001)
                p_.sub_(3e-4 * (m / 0.1) / ((v / 0.001).sqrt() + 1e-8))
                p_.grad = None

    sec, n = _cpu_time(step, budget_s, 1)
    rec("c5_gpt2_train_step", cfg.seq / sec, "tokens/s",
        f"fp32 torch autograd of the GPT-2-small step (12 layers, d 768, vocab 50257) on 1 of the 8 sequences "
        f"(1024 tokens) plus Adam over all parameters, {n} steps; tokens/s of that sample")
    return out


def run_sdpa(torch, np, K, args):
    from oracle import inputs

    B, H, D = 4, 16, 128
    scale = 1 / math.sqrt(D)
    seqs = [args.seq] if args.only == "headline" else [512, 1024, 2048, 4096, 8192, 16384]
    sweep = {}
    head = None
    for S in seqs:
        d = inputs.c3_sdpa(S)
        q, k, v = (dev_bf16(d[n], torch, np) for n in ("q", "k", "v"))
        del d
        o = torch.empty_like(q)
        steps = args.steps if S == args.seq else max(5, min(args.steps, 20))
        call = lambda: K.sdpa_fwd(q, k, v, scale, True, out=o)  # noqa: E731
        spin(torch, call, args.spinup if S == args.seq else min(args.spinup, 0.2))
        ms = time_launches(torch, call, steps, args.warmup)
        tf = sdpa_flops(B, H, S, D) / (ms * 1e-3) / 1e12
        sweep[str(S)] = {"ms": round(ms, 4), "tflops": round(tf, 2), "frac_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
        log(f"sdpa S={S}: {ms:.3f} ms  {tf:.1f} TFLOP/s  ({100*tf/PEAK_BF16_TFLOPS:.1f}% of bf16 peak)")
        if S == args.seq:
            head = (ms, tf, steps, o[0:1].clone())
        del q, k, v, o
        torch.cuda.empty_cache()
    return sweep, head


def run_fusions(torch, np, K, args):
    from oracle import inputs

    res = {}

    def rec(name, nbytes, fn, steps=20):
        ms = time_launches(torch, fn, steps, 3)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"ms": round(ms, 5), "bytes": int(nbytes), "gbs": round(gbs, 1),
                     "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"{name}: {ms*1e3:.1f} us  {gbs:.0f} GB/s ({100*gbs/PEAK_HBM_GBS:.1f}% of HBM peak)")

    d = inputs.c2_layernorm()
    x, g, b = (dev_bf16(d[n], torch, np) for n in ("x", "gamma", "beta"))
    rec("layernorm_8192x4096_bf16", 8192 * 4096 * 2 * 2 + 4096 * 2 * 2, lambda: K.layernorm(x, g, b, 1e-5))
    del x, g, b, d
    x = dev_bf16(inputs.c2_gelu()["x"], torch, np)
    y = torch.empty_like(x)
    rec("gelu_tanh_8192x16384_bf16", x.numel() * 4, lambda: K.gelu_tanh(x, out=y))
    del x, y
    x = dev_bf16(inputs.c2_reduce()["x"], torch, np)
    rec("reduce_sum_65536x1024_bf16", x.numel() * 2 + 65536 * 4, lambda: K.row_reduce(x, "sum"))
    rec("argmax_65536x1024_bf16", x.numel() * 2 + 65536 * 4, lambda: K.row_argmax(x, with_values=False))
    del x
    d = inputs.c4_indexing()
    table = dev_bf16(d["table_bf16"], torch, np)
    ids = torch.from_numpy(d["ids"]).cuda()
    rec("gather_32x2048_from_50257x768_bf16", 65536 * 4 + 2 * 65536 * 768 * 2, lambda: K.gather_rows(table, ids))
    tf = torch.from_numpy(d["table_f32"]).cuda()
    gr = torch.from_numpy(d["grads"]).cuda()
    out = torch.empty_like(tf)
    ws = torch.empty(int(K.lib().mk_scatter_add_workspace_bytes(50257, 65536)), dtype=torch.uint8, device="cuda")
    idf = ids.reshape(-1)
    rec("scatter_add_65536x768_into_50257x768_f32", 65536 * 768 * 4 + 65536 * 4 + 2 * 50257 * 768 * 4,
        lambda: K.scatter_add_rows(tf, idf, gr, out=out, workspace=ws))
    return res


# The GEMMs of one C5 step: (tag, out dtype, M, N, K, A layout, B layout).
# Layout "rm" = row-major [rows, cols] view, "t" = transposed view of the
# row-major [cols, rows] tensor (a unit stride along the other dimension).
C5_GEMMS = [
    ("qkv", "bf16", 8192, 2304, 768, "rm", "rm"), ("o", "bf16", 8192, 768, 768, "rm", "rm"),
    ("fc", "bf16", 8192, 3072, 768, "rm", "rm"), ("proj", "bf16", 8192, 768, 3072, "rm", "rm"),
    ("logits", "bf16", 8192, 50257, 768, "rm", "t"), ("dhf", "bf16", 8192, 768, 50257, "rm", "rm"),
    ("dwte", "f32", 50257, 768, 8192, "t", "rm"), ("dw_pr", "f32", 3072, 768, 8192, "t", "rm"),
    ("dg", "bf16", 8192, 3072, 768, "rm", "t"), ("dw_fc", "f32", 768, 3072, 8192, "t", "rm"),
    ("dh2", "bf16", 8192, 768, 3072, "rm", "t"), ("dw_o", "f32", 768, 768, 8192, "t", "rm"),
    ("datt", "bf16", 8192, 768, 768, "rm", "t"), ("dw_qkv", "f32", 768, 2304, 8192, "t", "rm"),
    ("dh", "bf16", 8192, 768, 2304, "rm", "t"),
]


def run_gemm(torch, np, K, args):
    """mk_gemm (hand-written MFMA) and mk_gemm_blas (rocBLAS) on the C5 step's
    15 GEMM shapes, and C1's two fp32 GEMMs (bias + ReLU, bias epilogues) on
    mk_gemm; TFLOP/s against the bf16 (2516.6) or fp32 (157.3) peak.  The
    fp32 weight-gradient shapes are also timed split along K as the C5 step
    runs them (mk_gemm_splitk, and rocBLAS with the same slices)."""
    from mi355x_pjrt.gpt2 import GPT2TrainStep
    from oracle import inputs

    res = {}
    g = torch.Generator(device="cuda").manual_seed(0)

    V = 50257
    Vp = (V + 7) // 8 * 8

    def mat(rows, cols, layout, dt):
        # the vocabulary dimension is stored with the padded row pitch the
        # C5 step uses (50264), so the vocabulary products see its layout
        r2, c2 = (rows, cols) if layout == "rm" else (cols, rows)
        pc = Vp if c2 == V else c2
        t = torch.randn(r2, pc, device="cuda", generator=g).to(dt)[:, :c2]
        return t if layout == "rm" else t.t()

    for tag, od, M, N, Kd, la, lb in C5_GEMMS:
        a, b = mat(M, Kd, la, torch.bfloat16), mat(Kd, N, lb, torch.bfloat16)
        odt = torch.float32 if od == "f32" else torch.bfloat16
        c = torch.empty(M, Vp if N == V else N, dtype=odt, device="cuda")[:, :N]
        fl = 2.0 * M * N * Kd
        row = {"M": M, "N": N, "K": Kd}
        for name, fn in (("mk_gemm", lambda: K.gemm(a, b, out_dtype=odt, out=c)),
                         ("rocblas", lambda: K.gemm_blas(a, b, out=c))):
            ms = time_launches(torch, fn, max(5, args.steps // 2), 3)
            row[name + "_tflops"] = round(fl / (ms * 1e-3) / 1e12, 1)
        row["mk_gemm_frac_peak"] = round(row["mk_gemm_tflops"] / PEAK_BF16_TFLOPS, 4)
        msg = f"gemm {tag} [{M}x{N}x{Kd}]: mk_gemm {row['mk_gemm_tflops']} TFLOP/s, rocBLAS {row['rocblas_tflops']}"
        if tag == "dhf":  # the C5 step splits it along the vocabulary (uneven slices, bf16 out)
            sp = GPT2TrainStep.DHF_SPLITS
            ms = time_launches(torch, lambda: K.gemm_splitk(a, b, sp, out=c, out_dtype=odt), max(5, args.steps // 2), 3)
            row["mk_gemm_splitk_tflops"] = round(fl / (ms * 1e-3) / 1e12, 1)
            row["splits"] = sp
            msg += f"; split {sp}: mk_gemm_splitk_typed {row['mk_gemm_splitk_tflops']}"
        row["c5_step_path"] = ("rocBLAS" if tag in GPT2TrainStep.BLAS_GEMMS else
                               "mk_gemm_splitk_typed" if tag == "dhf" else
                               "mk_gemm_splitk" if tag in GPT2TrainStep.DW_SPLITS else "mk_gemm")
        sp = GPT2TrainStep.DW_SPLITS.get(tag, 1)
        if sp > 1:  # the C5 step runs these fp32 weight gradients split along K
            for name, fn in (("mk_gemm_splitk", lambda: K.gemm_splitk(a, b, sp, out=c)),
                             ("rocblas_splitk", lambda: K.gemm_blas_splitk(a, b, sp, out=c))):
                ms = time_launches(torch, fn, max(5, args.steps // 2), 3)
                row[name + "_tflops"] = round(fl / (ms * 1e-3) / 1e12, 1)
            row["splits"] = sp
            msg += f"; split {sp}: mk_gemm_splitk {row['mk_gemm_splitk_tflops']}, rocBLAS {row['rocblas_splitk_tflops']}"
        res[tag] = row
        log(msg)
        del a, b, c
    res["c1_mlp_fp32"] = run_c1_pjrt(np, args)
    return res


def run_c1_pjrt(np, args):
    """Config C1 (fp32 MLP forward) as jaxlib runs it: the module compiled by
    jam (each product split along K into about 256 workgroups, bias / ReLU
    applied by the pass that sums the slices) and run through PJRT Execute on
    resident inputs; TFLOP/s against the fp32 MFMA peak (157.3)."""
    from mi355x_pjrt import modules, pjrt
    from oracle import inputs

    p = pjrt.Plugin()
    client = p.client()
    e = client.compile(modules.mlp())
    d = inputs.c1_mlp()
    bufs = [client.put(d[k]) for k in ("x", "w1", "b1", "w2", "b2")]
    for b in bufs:
        b.ready()
    run = pjrt_runner(p)
    run(e, bufs, 5)
    ms = run(e, bufs, max(20, args.steps))
    for b in bufs:
        b.destroy()
    e.destroy()
    client.close()
    fl = 2.0 * 256 * 1024 * 4096 * 2
    tf = fl / (ms * 1e-3) / 1e12
    log(f"C1 MLP fp32 through PJRT Execute: {ms*1e3:.1f} us, {tf:.1f} TFLOP/s ({100*tf/157.3:.1f}% of fp32 peak)")
    return {"ms": round(ms, 4), "tflops": round(tf, 2), "frac_peak_fp32": round(tf / 157.3, 4),
            "path": "PJRT Execute of the C1 module (jam: one gemm_splitk per layer, bias / ReLU in the slice sum)"}


def pjrt_runner(p):
    """run(exe, inputs, n): n executes queued back to back; host wall clock
    per execute (ms) until the last completion event."""

    def run(exe, inputs_, n):
        # each execution's outputs are dropped once the next one is queued,
        # as a loop that consumes its results does: the pool hands the freed
        # blocks back in stream order, so the steady state allocates nothing
        prev, ev = [], None
        t0 = time.perf_counter()
        for _ in range(n):
            if ev is not None:
                p.call("Event_Destroy", event=ev)
            o, ev = exe.execute(inputs_, wait="event")
            for b in prev:
                b.destroy()
            prev = o
        p.await_event(ev)
        el = time.perf_counter() - t0
        for b in prev:
            b.destroy()
        return el / n * 1e3

    return run


def run_pjrt_c5(np, args):
    """Only the jitted C5 step through the plugin (for profiling)."""
    from mi355x_pjrt import pjrt

    p = pjrt.Plugin()
    client = p.client()
    res = run_c5_jitted(np, p, client, pjrt_runner(p), args)
    client.close()
    return res


def run_pjrt(torch, np, args):
    """The plugin path: the C3 module at S=8192 compiled by jam and run
    through PJRT_LoadedExecutable_Execute with inputs resident in HBM (K
    executes queued back to back, host wall clock until the last completion
    event), and the per-Execute cost of a tiny module."""
    from mi355x_pjrt import modules, pjrt
    from oracle import bf16, inputs

    p = pjrt.Plugin()
    client = p.client()
    d = inputs.c3_sdpa(args.seq)
    e = client.compile(modules.sdpa(4, 16, args.seq, 128, True))
    bufs = [client.put(d[k], pjrt.BF16) for k in ("q", "k", "v")]
    for b in bufs:
        b.ready()

    run = pjrt_runner(p)
    # Executes first run for --spinup seconds on the same inputs (the clocks
    # leave whatever state the previous section left them in), then the
    # Execute path and the bare kernel (mk_sdpa_fwd on copies of the same
    # inputs, HIP events) are timed alternately, three rounds each, so the
    # per-Execute overhead is the difference of the two in one warm state
    from mi355x_pjrt import kernels as K
    t0 = time.time()
    while time.time() - t0 < max(args.spinup, 0.3):
        run(e, bufs, 10)
    qd, kd, vd = (torch.from_numpy(d[k].view(np.int16)).view(torch.bfloat16).cuda() for k in ("q", "k", "v"))
    od = torch.empty_like(qd)
    ex, bare = [], []
    for _ in range(3):
        run(e, bufs, args.warmup)
        ex.append(run(e, bufs, args.steps))
        bare.append(time_launches(torch, lambda: K.sdpa_fwd(qd, kd, vd, 1 / math.sqrt(128), True, out=od),
                                  args.steps, args.warmup))
    ms, ms_bare = sorted(ex)[1], sorted(bare)[1]
    del qd, kd, vd, od
    tf = sdpa_flops(4, 16, args.seq, 128) / (ms * 1e-3) / 1e12
    small = client.compile(modules.reduce_sum(4, 8))
    xb = client.put(bf16.to_bf16_bits(np.ones((4, 8), np.float32)), pjrt.BF16)
    run(small, [xb], 20)
    us = run(small, [xb], 200) * 1e3
    log(f"PJRT Execute, C3 S={args.seq}: {ms:.3f} ms/execute, {tf:.1f} TFLOP/s; tiny module {us:.1f} us/execute")
    for b in bufs + [xb]:
        b.destroy()
    e.destroy()
    small.destroy()
    res = {"sdpa_ms_per_execute": round(ms, 4), "sdpa_tflops": round(tf, 2),
           "sdpa_bare_kernel_ms_same_state": round(ms_bare, 4),
           "execute_overhead_frac": round(ms / ms_bare - 1, 4),
           "tiny_module_us_per_execute": round(us, 2)}
    res["c5_jitted_step"] = run_c5_jitted(np, p, client, run, args)
    client.close()
    return res


def run_c5_jitted(np, p, client, run, args):
    """The C5 training step as one jitted StableHLO module (train_hlo:
    forward, reverse-mode gradients, Adam) compiled by jam and run through
    Execute on resident inputs: the same work as the hand-scheduled step,
    lowered by jam's pattern matchers (flash attention forward and backward,
    LayerNorm forward and backward, cross-entropy, biased products) and
    generated elementwise kernels.  Executes are queued back to back (each
    one's outputs dropped after the next is queued); up to 20 of them are
    timed after two untimed ones, so the host's latency to the first launch
    is spread over the timed steps."""
    from mi355x_pjrt import gpt2, train_hlo

    cfg = gpt2.GPT2Config()
    t0 = time.perf_counter()
    e = client.compile(train_hlo.gpt2_train_step(cfg))
    compile_s = time.perf_counter() - t0
    params = gpt2.init_params(cfg, 0)
    names = [n for n, _ in cfg.param_shapes()]
    rng = np.random.default_rng(5000)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq)).astype(np.int32)
    host = ([params[n] for n in names] + [np.zeros_like(params[n]) for n in names] * 2 +
            [ids, np.roll(ids, -1, axis=1), np.float32(3e-4), np.float32(1 / (1 - 0.9)), np.float32(1 / (1 - 0.999))])
    bufs = [client.put(np.asarray(a)) for a in host]
    for b in bufs:
        b.ready()
    n = max(2, min(args.steps, 20))
    run(e, bufs, 2)
    ms = run(e, bufs, n)
    for b in bufs:
        b.destroy()
    e.destroy()
    fl = cfg.flops_per_step()
    log(f"C5 jitted step through PJRT Execute: {ms:.2f} ms/step, {cfg.tokens / (ms * 1e-3):.0f} tokens/s "
        f"(compile {compile_s:.2f} s)")
    return {"workload": "C5 GPT-2-small training step as one jitted module (B=8 S=1024), bf16 products, fp32 "
                        "elsewhere, attention fwd+bwd matched to the flash kernels", "ms_per_step": round(ms, 3),
            "tokens_per_s": round(cfg.tokens / (ms * 1e-3), 1), "model_tflops": round(fl / (ms * 1e-3) / 1e12, 2),
            "steps": n, "compile_s": round(compile_s, 3)}


def run_c5(torch, np, args):
    """C5 training step, graph-replayed: W untimed replays, then K timed
    replays between HIP events on the step's stream."""
    from mi355x_pjrt import gpt2

    cfg = gpt2.GPT2Config()
    stream = torch.cuda.Stream()
    step = gpt2.GPT2TrainStep(cfg, seed=0, stream=stream)
    rng = np.random.default_rng(5000)
    ids = rng.integers(0, cfg.vocab, (cfg.batch, cfg.seq))
    step.set_batch(ids, np.roll(ids, -1, axis=1))
    step.step()  # eager first step (library handles), then capture
    torch.cuda.synchronize()
    loss_first = step.loss_value()
    step.capture()
    for _ in range(args.warmup):
        step.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    fl = cfg.flops_per_step()
    res = {"workload": "C5 GPT-2-small training step (forward + backward + Adam), B=8 S=1024 d=768 L=12 H=12 "
                       "V=50257, bf16 activations, fp32 master/Adam, one HIP graph per step",
           "ms_per_step": round(ms, 4), "tokens_per_s": round(cfg.tokens / (ms * 1e-3), 1),
           "model_tflops": round(fl / (ms * 1e-3) / 1e12, 2), "flops_per_step": fl,
           "mfu": round(fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), "steps": args.steps,
           "warmup": args.warmup, "loss_step1": round(loss_first, 4),
           "loss_last": round(step.loss_value(), 4), "params": step.n_params,
           "data": "synthetic: numpy PCG64 token ids U[0,V), labels = ids shifted by one; N(0,0.02) init"}
    log(f"C5 step: {ms:.3f} ms, {res['tokens_per_s']:.0f} tokens/s, {res['model_tflops']:.1f} TFLOP/s, "
        f"MFU {100 * res['mfu']:.1f}%")
    del step
    torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU: multi-GPU execution "
                          "(RCCL collectives) is out of scope; run with --gpus 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device"}))
        sys.exit(1)
    from mi355x_pjrt import kernels as K

    K.lib()
    torch.cuda.init()
    if args.only == "calib":
        # plain copy of a known size: calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE
        n = 128 << 20  # 128 Mi float32 = 512 MiB read + 512 MiB write per launch
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        ms = time_launches(torch, lambda: K.copy_strided(src), 5, 1)
        print(json.dumps({"calib_copy_bytes_read": n * 4, "calib_copy_bytes_written": n * 4,
                          "ms": round(ms, 4), "gbs": round(2 * n * 4 / (ms * 1e-3) / 1e9, 1)}))
        return
    if args.only == "c5":
        print(json.dumps({"training_step": run_c5(torch, np, args)}))
        return
    if args.only == "gemm":
        print(json.dumps({"gemm": run_gemm(torch, np, K, args)}))
        return
    if args.only == "pjrt":
        print(json.dumps({"pjrt": run_pjrt(torch, np, args)}))
        return
    if args.only == "c1":
        print(json.dumps({"c1_mlp_fp32": run_c1_pjrt(np, args)}))
        return
    if args.only == "c5jit":
        print(json.dumps({"c5_jitted_step": run_pjrt_c5(np, args)}))
        return
    sweep, head, fusions = {}, None, {}
    spin_up(torch, np, K, args)
    if args.only in (None, "sdpa", "headline"):
        sweep, head = run_sdpa(torch, np, K, args)
    if args.only in (None, "fusions"):
        fusions = run_fusions(torch, np, K, args)
    if head is None:
        print(json.dumps({"fusions": fusions}))
        return
    c5 = run_c5(torch, np, args) if args.only is None else None
    plugin = run_pjrt(torch, np, args) if args.only is None else None
    gemm = run_gemm(torch, np, K, args) if args.only is None else None
    ms, tf, steps, o0 = head
    S = args.seq
    cpu = None if args.no_cpu else cpu_baseline_sdpa(torch, np, S, args.cpu_seconds, gpu_out=o0)
    cpu_other = None if args.no_cpu or args.only is not None else cpu_baselines(torch, np, args.cpu_seconds / 3)
    traffic = read_traffic(f"sdpa_fwd_causal_b4h16d128_s{S}_traffic")
    line = {
        "metric": "SDPA TFLOP/s vs seq len (512-16384) & % MFMA peak; fusion GB/s % HBM peak",
        "value": round(tf, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "spinup_s": args.spinup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: numpy PCG64 N(0,1)/sqrt(128) bf16, seeds 3000-3002",
        "config": {"workload": f"C3 causal SDPA forward B=4 H=16 S={S} D=128 bf16 (mk_sdpa_fwd)",
                   "batch": 4, "heads": 16, "seq_len": S, "head_dim": 128, "causal": True,
                   "flops_per_step": sdpa_flops(4, 16, S, 128)},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "cpu_baselines_other_configs": cpu_other,
        "sweep": sweep,
        "fusions": fusions,
        "training_step": c5,
        "pjrt_execute": plugin,
        "gemm": gemm,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
