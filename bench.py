#!/usr/bin/env python3
"""Benchmark of the algebraic-extra hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]

A step is one forward+backward of the guarded asinh-power causal attention
(flash_attention(kind="asinh", n=16, c=8, range_guard=True), the model's
call, model.py:145-150) at BASELINE.json configs[1]: B=8, H=12, T=2048,
D=64, bf16, q/k QK-normalised N(0,1), v and dO N(0,1), synthetic and seeded.
`value` is that step's throughput in TFLOP/s under the reference's FLOP
convention (bench_attention.py:50,65: fwd+bwd = 3.5 * 4*B*H*T^2*D/2).

One JSON line is printed. Besides the contract keys it carries:
  roofline      the dominant kernel (attention backward) timed with HIP events
                that libalgx records as part of that kernel's own dispatch
                (hipExtLaunchKernel, on the stream it runs on) during the timed
                steps, against the MI355X dense bf16 MFMA peak;
  cpu_baseline  the reference's dense algebraic attention restated in torch
                CPU float32 (oracle/cpu_baseline.py) on a bounded sample;
  secondary     configs[3] attention (H=16), the fused LM head + loss at
                configs[2] (tokens/s, TFLOP/s by bench_head.py:36) and the
                QK RMS-norm kernels at configs[3] (GB/s against 8 TB/s).
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "algebraic-extra_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "asinh-attn fwd+bwd TFLOP/s (S=2048,D=64 bf16); fused-head tokens/s; %roofline"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (no sparsity)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def attn_flops_fwd(B, H, T, D):
    return 4.0 * B * H * T * T * D / 2.0      # causal, bench_attention.py:50


def head_flops(N, d, V):
    return 3 * 2.0 * N * d * V                # logits, dh, dE; bench_head.py:36


def make_attention_inputs(B, H, T, D, seed, dev, qk_norm=True):
    """q, k, v (leaves) and dO, bf16 N(0, 1); q and k QK-normalised as the
    model's attention inputs are, or raw N(0, 1) as the reference's harness
    draws them (bench_attention.py:47-48) with qk_norm=False."""
    import torch
    gen = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn((B, H, T, D), device=dev, generator=gen)
    k = torch.randn((B, H, T, D), device=dev, generator=gen)
    if qk_norm:
        q = q * torch.rsqrt((q * q).mean(-1, keepdim=True) + 1e-5)
        k = k * torch.rsqrt((k * k).mean(-1, keepdim=True) + 1e-5)
    q, k = q.bfloat16(), k.bfloat16()
    v = torch.randn((B, H, T, D), device=dev, generator=gen).bfloat16()
    do = torch.randn((B, H, T, D), device=dev, generator=gen).bfloat16()
    return [x.requires_grad_(True) for x in (q, k, v)] + [do]


class Probe:
    """HIP events that libalgx records with one named kernel's dispatch
    (algx_set_probe): one (start, stop) pair per timed step."""

    def __init__(self, which, count):
        import torch
        from algebraic_amd import _lib
        self._lib = _lib
        self.which = _lib.PROBE[which]
        self.pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(count)]
        for a, b in self.pairs:          # materialise the underlying hipEvents
            a.record()
            b.record()
        torch.cuda.synchronize()

    def arm(self, i):
        a, b = self.pairs[i]
        self._lib.call("algx_set_probe", self.which, a.cuda_event, b.cuda_event)

    def disarm(self):
        self._lib.call("algx_set_probe", 0, None, None)

    def mean_ms(self, count=None):
        pairs = self.pairs[:count] if count else self.pairs
        return sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)


SETTLE_S = 1.0   # untimed running before the warmup steps: GPU clocks settle


def time_steps(step, steps, warmup, probe=None, settle_s=SETTLE_S):
    """Wall time per step over `steps` after `warmup`; probe armed per step.

    Before the `warmup` steps the step runs untimed for `settle_s` seconds,
    so the timed steps see the GPU at its steady clocks rather than ramping
    out of idle (a cold MI355X runs the first ~second of work measurably
    slower)."""
    import torch
    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        for _ in range(8):       # back to back, as the timed steps run
            step()
        torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        if probe is not None:
            probe.arm(i)
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    if probe is not None:
        probe.disarm()
    return dt


def bench_attention(B, H, T, D, steps, warmup, dev, kind="asinh", kw=None, sink=False,
                    qk_norm=True):
    """One fwd+bwd step of flash_attention; `kw` replaces the default call
    (the model's guarded n=16, c=8 asinh, or plain softmax), `sink` passes a
    zero sink logit of shape (1, H, 1, 1) as the reference's harness does
    (bench_attention.py:49)."""
    import torch
    from algebraic_amd.kernels import flash_attention
    q, k, v, do = make_attention_inputs(B, H, T, D, 1, dev, qk_norm=qk_norm)
    if kw is None:
        kw = (dict(kind="asinh", n=16, c=8.0, range_guard=True) if kind == "asinh"
              else dict(kind="softmax"))
    s = torch.zeros((1, H, 1, 1), dtype=torch.float32, device=dev) if sink else None

    def step():
        o = flash_attention(q, k, v, s, **kw)
        torch.autograd.grad(o, (q, k, v), do)

    bwd_probe = Probe("attn_bwd", steps)
    dt = time_steps(step, steps, warmup, bwd_probe)
    fwd_probe = Probe("attn_fwd", steps)
    time_steps(step, steps, 1, fwd_probe)
    f_fwd = attn_flops_fwd(B, H, T, D)
    return {
        "ms_per_step": dt * 1e3,
        "tflops": 3.5 * f_fwd / dt / 1e12,
        "bwd_kernel_ms": bwd_probe.mean_ms(),
        "fwd_kernel_ms": fwd_probe.mean_ms(),
        "bwd_flops": 2.5 * f_fwd,
        "fwd_flops": f_fwd,
    }


def bench_head(steps, warmup, dev, N=16384, d=768, V=50304, kind="alg_ce", n=8, c=2.0,
               library=True):
    import torch
    from algebraic_amd.kernels import fused_head
    gen = torch.Generator(device=dev).manual_seed(2)
    h = torch.randn((N, d), device=dev, generator=gen).bfloat16().requires_grad_(True)
    E = (torch.randn((V, d), device=dev, generator=gen) * 0.02).bfloat16().requires_grad_(True)
    t = torch.randint(0, V, (N,), device=dev, generator=gen, dtype=torch.int64)

    def step():
        obj, _ = fused_head(h, E, t, kind=kind, n=n, c=c)
        torch.autograd.grad(obj, (h, E))

    dt = time_steps(step, steps, warmup)
    # Kernel split (HIP events recorded with each kernel's dispatch): the
    # forward statistics, the dz recompute and the grouped dh + dE GEMMs.
    split = {}
    for name in ("head_fwd", "head_dz", "head_de"):
        pr = Probe(name, steps)
        time_steps(step, steps, 1, pr, settle_s=0.0)
        split[{"head_fwd": "fwd_ms", "head_dz": "dz_ms", "head_de": "dh_dE_ms"}[name]] = pr.mean_ms()
    flops = head_flops(N, d, V)
    return {"workload": f"N={N},d={d},V={V},{kind} n={n} c={c}", "ms_per_step": dt * 1e3,
            "tokens_per_s": N / dt, "tflops": flops / dt / 1e12,
            "frac": flops / dt / 1e12 / PEAK_BF16_TFLOPS, **split,
            **({"library_gemm_tflops": library_gemm_rates(h.detach(), E.detach())}
               if library else {})}


def library_gemm_rates(h, E, iters=10):
    """The rate torch's GEMM library (hipBLASLt / rocBLAS, default heuristics)
    reaches on the head's three products as plain bf16 GEMMs: the logits
    z = h E^T (written out, which the fused kernels never do), dh = dz E and
    dE = dz^T h with a [N, V] dz. A ceiling reference for the head's own
    MFMA loops at the same shapes, not part of the timed step."""
    import torch
    N, d = h.shape
    V = E.shape[0]
    dz = torch.empty((N, V), device=h.device, dtype=torch.bfloat16).normal_(0.0, 1e-3)
    cases = {"logits": lambda: torch.mm(h, E.t()), "dh": lambda: torch.mm(dz, E),
             "dE": lambda: torch.mm(dz.t(), h)}
    flops = 2.0 * N * d * V
    out = {}
    for name, f in cases.items():
        for _ in range(2):
            f()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            f()
        e.record()
        torch.cuda.synchronize()
        out[name] = round(flops / (s.elapsed_time(e) / iters * 1e-3) / 1e12, 1)
    del dz
    torch.cuda.empty_cache()
    return out


def bench_harness_variants(steps, warmup, dev):
    """The reference harness's attention sweep at configs[1]'s shape
    (bench_attention.py:75-80): softmax with a zero sink, and asinh n=16,
    c=16 shifted (exact rho), shifted + fast rho and unshifted + fast rho,
    each with a zero sink, on raw N(0, 1) bf16 q, k, v as the harness draws
    them; fwd+bwd step time and the forward and backward kernel times."""
    B, H, T, D = 8, 12, 2048, 64
    cases = {"softmax+sink": dict(kind="softmax")}
    for shift, fast in ((True, False), (True, True), (False, True)):
        name = f"asinh16/16 {'shift' if shift else 'noshift'}{'+fast' if fast else ''}"
        cases[name] = dict(kind="asinh", n=16, c=16.0, shift=shift, fast_rho=fast)
    out = {"workload": "bench_attention.py:75-80 at B=8,H=12,T=2048,D=64 bf16, raw N(0,1) "
                       "q,k,v, zero sink (1,H,1,1)"}
    for name, kw in cases.items():
        a = bench_attention(B, H, T, D, steps, warmup, dev, kw=kw, sink=True, qk_norm=False)
        out[name] = {"ms_per_step": round(a["ms_per_step"], 4), "tflops": round(a["tflops"], 2),
                     "frac": round(a["tflops"] / PEAK_BF16_TFLOPS, 4),
                     "fwd_kernel_ms": round(a["fwd_kernel_ms"], 4),
                     "bwd_kernel_ms": round(a["bwd_kernel_ms"], 4)}
    return out


class CacheFlush:
    """A 1 GiB buffer read between timed calls: it evicts the 256 MB Infinity
    Cache (and the L2s), so the next call's operands come from HBM. It is
    read, not written, so the cache holds clean lines afterwards and no
    write-back of the flush itself overlaps the timed call."""

    def __init__(self, dev):
        import torch
        self.buf = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)

    def __call__(self):
        self.buf.amax()


def bench_qknorm(steps, warmup, dev):
    """QK-norm over the attention's q and k ([8, 2048, 16, 64] bf16 each) in
    one launch each way (qk_rms_norm_pair); the per-tensor calls are timed
    beside it. Each is timed warm (the step repeated back to back: its
    134 MB / 201 MB of operands largely stay in the 256 MB Infinity Cache)
    and cold (a 1 GiB read between steps), next to a plain device copy of
    the same bytes (torch copy_, one read and one write per element) as the
    ceiling a streaming kernel of that size reaches in the same run."""
    import torch
    from algebraic_amd.kernels import qk_rms_norm, qk_rms_norm_pair
    gen = torch.Generator(device=dev).manual_seed(3)
    shape = (8, 2048, 16, 64)
    xs = [torch.randn(shape, device=dev, generator=gen).bfloat16().requires_grad_(True)
          for _ in range(2)]
    gains = [(1 + 0.01 * torch.randn(64, device=dev, generator=gen)).requires_grad_(True)
             for _ in range(2)]
    dys = [torch.randn(shape, device=dev, generator=gen).bfloat16() for _ in range(2)]

    def pair_step():
        yq, yk = qk_rms_norm_pair(xs[0], xs[1], gains[0], gains[1])
        torch.autograd.grad((yq, yk), (xs[0], xs[1], gains[0], gains[1]), dys)

    def single_step():
        for x, g, dy in zip(xs, gains, dys):
            torch.autograd.grad(qk_rms_norm(x, g), (x, g), dy)

    fp, bp = Probe("qknorm_fwd", steps), Probe("qknorm_bwd", steps)
    time_steps(pair_step, steps, warmup, fp)
    time_steps(pair_step, steps, 1, bp)
    sfp, sbp = Probe("qknorm_fwd", steps), Probe("qknorm_bwd", steps)
    time_steps(single_step, steps, warmup, sfp, settle_s=0.0)
    time_steps(single_step, steps, 1, sbp, settle_s=0.0)
    elems = 2 * xs[0].numel()
    # Each probe brackets the row kernel of one launch (the dgain finish is a
    # separate 128-block launch); the per-tensor probe holds the k call.
    fwd_bytes, bwd_bytes = elems * 4, elems * 6
    f_ms, b_ms = fp.mean_ms(), bp.mean_ms()
    out = {"workload": "q,k each [8,2048,16,64] bf16, D=64 rows, one launch for both",
           "fwd_us": f_ms * 1e3, "fwd_gbs": fwd_bytes / f_ms / 1e6,
           "bwd_us": b_ms * 1e3, "bwd_gbs": bwd_bytes / b_ms / 1e6,
           "fwd_frac": fwd_bytes / f_ms / 1e6 / PEAK_HBM_GBS,
           "bwd_frac": bwd_bytes / b_ms / 1e6 / PEAK_HBM_GBS,
           "per_tensor_fwd_us": sfp.mean_ms() * 1e3, "per_tensor_bwd_us": sbp.mean_ms() * 1e3}
    out["per_tensor_fwd_frac"] = fwd_bytes / 2 / sfp.mean_ms() / 1e6 / PEAK_HBM_GBS
    out["per_tensor_bwd_frac"] = bwd_bytes / 2 / sbp.mean_ms() / 1e6 / PEAK_HBM_GBS

    # Cold: the Infinity Cache flushed before every timed call.
    flush = CacheFlush(dev)

    def cold(step, probe, n):
        for i in range(n):
            flush()
            probe.arm(i)
            step()
        probe.disarm()
        torch.cuda.synchronize()

    for name, step, nbytes in (("pair", pair_step, (fwd_bytes, bwd_bytes)),
                               ("per_tensor", single_step, (fwd_bytes / 2, bwd_bytes / 2))):
        cf, cb = Probe("qknorm_fwd", steps), Probe("qknorm_bwd", steps)
        cold(step, cf, steps)
        cold(step, cb, steps)
        out[f"cold_{name}_fwd_us"] = cf.mean_ms() * 1e3
        out[f"cold_{name}_fwd_frac"] = nbytes[0] / cf.mean_ms() / 1e6 / PEAK_HBM_GBS
        out[f"cold_{name}_bwd_us"] = cb.mean_ms() * 1e3
        out[f"cold_{name}_bwd_frac"] = nbytes[1] / cb.mean_ms() / 1e6 / PEAK_HBM_GBS

    # Plain-copy ceilings at the per-tensor and pair sizes (67.1 / 134.2 MB
    # moved), warm and cold, event-timed per call.
    for name, n in (("per_tensor", xs[0].numel()), ("pair", 2 * xs[0].numel())):
        src = torch.ones(n, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for tag, pre in (("warm", None), ("cold", flush)):
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(steps)]
            for _ in range(3):
                dst.copy_(src)
            for a, b in ev:
                if pre is not None:
                    pre()
                a.record()
                dst.copy_(src)
                b.record()
            torch.cuda.synchronize()
            ms = sum(a.elapsed_time(b) for a, b in ev) / steps
            out[f"copy_{name}_{tag}_us"] = ms * 1e3
            out[f"copy_{name}_{tag}_frac"] = 4 * n / ms / 1e6 / PEAK_HBM_GBS
        del src, dst
    del flush
    torch.cuda.empty_cache()
    return out


def bench_elementwise(steps, warmup, dev):
    """rms_norm with a gain over 8 x 2048 rows of d_model = 1024 (the 350M
    model's ln1/ln2), and the fused alu_glu over its (8 x 2048, d_ff = 2688)
    feed-forward activations: kernel time from the probes, HBM bytes as the
    operands each kernel must move once."""
    import torch
    from algebraic_amd.algebraic import alu_glu, rms_norm
    gen = torch.Generator(device=dev).manual_seed(4)
    rows, d, dff = 16384, 1024, 2688
    x = torch.randn((rows, d), device=dev, generator=gen).bfloat16().requires_grad_(True)
    g = (1 + 0.1 * torch.randn(d, device=dev, generator=gen)).requires_grad_(True)
    dy = torch.randn((rows, d), device=dev, generator=gen).bfloat16()
    gate = torch.randn((rows, dff), device=dev, generator=gen).bfloat16().requires_grad_(True)
    up = torch.randn((rows, dff), device=dev, generator=gen).bfloat16().requires_grad_(True)
    dout = torch.randn((rows, dff), device=dev, generator=gen).bfloat16()

    def norm_step():
        torch.autograd.grad(rms_norm(x, g), (x, g), dy)

    def glu_step():
        torch.autograd.grad(alu_glu(gate, up, 1.0), (gate, up), dout)

    out = {"workload": f"rms_norm [{rows},{d}] bf16 + f32 gain; alu_glu [{rows},{dff}] bf16"}
    for name, step, elems, fb, bb in (("rms_norm", norm_step, rows * d, 4, 6),
                                      ("alu_glu", glu_step, rows * dff, 6, 10)):
        probe = "rms_norm" if name == "rms_norm" else "alu"
        fp, bp = Probe(probe + "_fwd", steps), Probe(probe + "_bwd", steps)
        time_steps(step, steps, warmup, fp)
        time_steps(step, steps, 1, bp)
        f_ms, b_ms = fp.mean_ms(), bp.mean_ms()
        out.update({f"{name}_fwd_us": f_ms * 1e3,
                    f"{name}_fwd_gbs": elems * fb / f_ms / 1e6,
                    f"{name}_fwd_frac": elems * fb / f_ms / 1e6 / PEAK_HBM_GBS,
                    f"{name}_bwd_us": b_ms * 1e3,
                    f"{name}_bwd_gbs": elems * bb / b_ms / 1e6,
                    f"{name}_bwd_frac": elems * bb / b_ms / 1e6 / PEAK_HBM_GBS})
    return out


def model_flops_per_token(cfg, T):
    """Training FLOPs per token without rematerialisation: 6 x the block and
    head parameters' MACs, plus 3.5 x the causal attention forward
    (2 H T D per layer and token)."""
    d, f, L, V, H, D = cfg.d_model, cfg.d_ff, cfg.n_layers, cfg.vocab_size, cfg.n_heads, cfg.head_dim
    dense = L * (4 * d * d + 3 * d * f) + d * V
    return 6 * dense + 3.5 * L * 2 * H * T * D


def bench_model(preset, steps, warmup, dev, B=8, T=2048, V=50304, remat=True, optimizer=False):
    """one forward + backward of the 350M preset (d 1024, 24 layers,
    16 heads of 64, d_ff 2688, V 50304) on B x T random tokens, random-init
    weights, bf16; parameter gradients are produced (no optimiser update).
    remat=True recomputes each block in the backward as the reference's
    default LMConfig does; remat=False keeps the activations (they fit in HBM
    at this size many times over). optimizer=True adds the reference trainer's
    default update, Muon on the layer matrices + AdamW on the rest
    (optimizers.py:118-246, lr 2e-3 as configs/comparison_350m.json), to
    every step: a full training step."""
    import torch
    from algebraic_amd import config, model
    # Plain library GEMMs: torch's TunableOp picks, per projection shape, the
    # fastest hipBLASLt or rocBLAS solution recorded for this ROCm/torch build
    # (selection only: no tuning runs here; unknown shapes keep the default).
    table = os.path.join(os.path.dirname(os.path.abspath(__file__)), "algebraic-extra_amd",
                         "algebraic_amd", "gemm_tuning_gfx950.csv")
    if os.path.exists(table):
        import tempfile
        torch.cuda.tunable.enable(True)
        torch.cuda.tunable.tuning_enable(False)
        # results are read from the table; anything written back goes to /tmp
        torch.cuda.tunable.set_filename(os.path.join(tempfile.gettempdir(),
                                                     f"algx_tunableop_{os.getpid()}.csv"))
        torch.cuda.tunable.read_file(table)
    cfg = config.build(preset, "350m", vocab_size=V, seq_len=T, attn_impl="flash",
                       head_impl="fused", remat=remat)
    params = model.init_params(cfg, seed=0, device=dev)
    leaves = list(model._leaves(params))
    gen = torch.Generator(device=dev).manual_seed(5)
    tok = torch.randint(0, V, (B, T + 1), generator=gen, device=dev)
    x, y = tok[:, :-1].contiguous(), tok[:, 1:].contiguous()
    tables = model.position_tables(cfg, T, device=dev)

    opt = None
    if optimizer:
        from algebraic_amd import optimizers
        init_fn, step_fn = optimizers.get_optimizer("muon_adamw", 2e-3, weight_decay=0.1)
        opt = [init_fn(params), 0]
        mask = model.decay_mask(params)

    def step():
        for t in leaves:
            t.grad = None
        obj, _ = model.train_objective(params, x, y, cfg, tables)
        obj.backward()
        if opt is not None:
            step_fn(opt[1], params, optimizers.grads_of(params), opt[0], mask)
            opt[1] += 1

    fpt = model_flops_per_token(cfg, T)
    torch.cuda.reset_peak_memory_stats()
    dt = time_steps(step, steps, warmup)
    what = "train step (fwd+bwd+Muon/AdamW)" if optimizer else "fwd+bwd"
    out = {"workload": f"configs[4] {preset} 350M {what}, B={B}, T={T}, V={V}, bf16, "
                       f"{'remat' if remat else 'no remat'}",
           "peak_hbm_gb": torch.cuda.max_memory_allocated() / 1e9,
           "ms_per_step": dt * 1e3, "tokens_per_s": B * T / dt,
           "tflops": fpt * B * T / dt / 1e12, "flops_per_token": fpt,
           "frac": fpt * B * T / dt / 1e12 / PEAK_BF16_TFLOPS,
           "params": model.count_params(params)}
    out["gemm_selection"] = "tunableop table" if torch.cuda.tunable.is_enabled() else "default"
    torch.cuda.tunable.enable(False)
    del params, leaves
    torch.cuda.empty_cache()
    return out


def bwd_counters():
    """Counter figures of the attention-backward kernel recorded from
    rocprofv3 --pmc runs in profiles/attn_bwd_traffic.json (HBM bytes per
    launch from FETCH_SIZE + WRITE_SIZE, MFMA / VALU / LDS busy fractions);
    empty when that summary is absent."""
    path = os.path.join(ROOT, "profiles", "attn_bwd_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def cpu_baseline(B, H, T, D, heads=None, runs=6):
    # The whole configs[1] workload, twice over (about 10 s on 16 host cores),
    # split into `runs` equal runs; the rate is the median run's.
    heads = heads or 2 * B * H
    from oracle.cpu_baseline import time_attention_fwd_bwd
    times, threads = time_attention_fwd_bwd(T=T, D=D, heads=heads)
    per_run = heads // runs
    run_secs = sorted(sum(times[i * per_run:(i + 1) * per_run]) for i in range(runs))
    med = 0.5 * (run_secs[(runs - 1) // 2] + run_secs[runs // 2])
    per_head = 3.5 * 4.0 * T * T * D / 2.0
    return {"value": per_run * per_head / med / 1e12, "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{heads} (b,h)-head fwd+bwd passes ({heads / (B * H):g}x the configs[1] "
                      f"workload of {B * H} heads) in {runs} runs of {per_run}, median run "
                      f"{med:.2f} s (all {sum(times):.1f} s); dense algebraic.asinh_attention "
                      f"fwd + autograd bwd in torch-CPU float32"}


def calibrate_copy(dev):
    """One plain 256 MiB device copy: the scale reference for the FETCH_SIZE /
    WRITE_SIZE counters of a rocprofv3 --pmc run (it must read 262144 KiB and
    write 262144 KiB)."""
    import torch
    src = torch.ones(128 << 20, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def run_once(which, dev, steps=3):
    """`steps` untimed steps of one benchmark workload (for counter passes)."""
    import torch
    if which in ("attn", "attn16"):
        from algebraic_amd.kernels import flash_attention
        H = 12 if which == "attn" else 16
        q, k, v, do = make_attention_inputs(8, H, 2048, 64, 1, dev)
        for _ in range(steps):
            o = flash_attention(q, k, v, kind="asinh", n=16, c=8.0, range_guard=True)
            torch.autograd.grad(o, (q, k, v), do)
    elif which == "attn_harness":
        # bench_attention.py:75-80's four variants at configs[1], zero sink
        from algebraic_amd.kernels import flash_attention
        q, k, v, do = make_attention_inputs(8, 12, 2048, 64, 1, dev, qk_norm=False)
        sink = torch.zeros((1, 12, 1, 1), dtype=torch.float32, device=dev)
        cases = [dict(kind="softmax")] + [
            dict(kind="asinh", n=16, c=16.0, shift=sh, fast_rho=fa)
            for sh, fa in ((True, False), (True, True), (False, True))]
        for kw in cases:
            for _ in range(steps):
                o = flash_attention(q, k, v, sink, **kw)
                torch.autograd.grad(o, (q, k, v), do)
    elif which == "head":
        from algebraic_amd.kernels import fused_head
        N, d, V = 16384, 768, 50304
        gen = torch.Generator(device=dev).manual_seed(2)
        h = torch.randn((N, d), device=dev, generator=gen).bfloat16().requires_grad_(True)
        E = (torch.randn((V, d), device=dev, generator=gen) * 0.02).bfloat16().requires_grad_(True)
        t = torch.randint(0, V, (N,), device=dev, generator=gen, dtype=torch.int64)
        for _ in range(steps):
            obj, _ = fused_head(h, E, t, kind="alg_ce", n=8, c=2.0)
            torch.autograd.grad(obj, (h, E))
    else:
        from algebraic_amd.kernels import qk_rms_norm_pair
        gen = torch.Generator(device=dev).manual_seed(3)
        shape = (8, 2048, 16, 64)
        xs = [torch.randn(shape, device=dev, generator=gen).bfloat16().requires_grad_(True)
              for _ in range(2)]
        gains = [(1 + 0.01 * torch.randn(64, device=dev, generator=gen)).requires_grad_(True)
                 for _ in range(2)]
        dys = [torch.randn(shape, device=dev, generator=gen).bfloat16() for _ in range(2)]
        for _ in range(steps):
            yq, yk = qk_rms_norm_pair(xs[0], xs[1], gains[0], gains[1])
            torch.autograd.grad((yq, yk), (xs[0], xs[1], gains[0], gains[1]), dys)
    torch.cuda.synchronize()


def read_sclk_mhz():
    """Current shader clock of GPU 0 from rocm-smi (None when unavailable)."""
    import re
    import subprocess
    try:
        out = subprocess.run(["rocm-smi", "--showclocks", "--json"], capture_output=True,
                             text=True, timeout=5).stdout
        for card in json.loads(out).values():
            for key, val in card.items():
                if "sclk clock speed" in key:
                    return float(re.sub(r"[^0-9.]", "", str(val)))
    except Exception:
        return None
    return None


def bench_clock(dev, seconds=3.0):
    """Hot-path steps run back to back for `seconds` each while rocm-smi
    samples the shader clock: the configs[1] attention step (fwd + bwd) and
    the configs[2] fused-head step (forward statistics, dz, dh + dE), each on
    the benchmark's inputs and on all-zero inputs, and the library's plain
    GEMM of the head's logits shape beside them. Under the benchmark's inputs
    these steps run at the board's power limit, below the maximum clock, and
    the clock depends on the data the MFMAs multiply."""
    import threading
    import torch
    from algebraic_amd.kernels import flash_attention, fused_head

    def attention(zero):
        q, k, v, do = make_attention_inputs(8, 12, 2048, 64, 1, dev)
        if zero:
            with torch.no_grad():
                for x in (q, k, v, do):
                    x.zero_()

        def step():
            o = flash_attention(q, k, v, kind="asinh", n=16, c=8.0, range_guard=True)
            torch.autograd.grad(o, (q, k, v), do)
        return step

    def head(zero):
        gen = torch.Generator(device=dev).manual_seed(2)
        N, d, V = 16384, 768, 50304
        h = torch.randn((N, d), device=dev, generator=gen).bfloat16()
        E = (torch.randn((V, d), device=dev, generator=gen) * 0.02).bfloat16()
        if zero:
            h.zero_()
            E.zero_()
        h.requires_grad_(True)
        E.requires_grad_(True)
        t = torch.randint(0, V, (N,), device=dev, generator=gen, dtype=torch.int64)

        def step():
            obj, _ = fused_head(h, E, t, kind="alg_ce", n=8, c=2.0)
            torch.autograd.grad(obj, (h, E))
        return step

    def library_logits():
        gen = torch.Generator(device=dev).manual_seed(2)
        h = torch.randn((16384, 768), device=dev, generator=gen).bfloat16()
        E = (torch.randn((50304, 768), device=dev, generator=gen) * 0.02).bfloat16()
        return lambda: torch.mm(h, E.t())

    cases = {"attention_random": (lambda: attention(False), 50),
             "attention_zero": (lambda: attention(True), 50),
             "head_random": (lambda: head(False), 5),
             "head_zero": (lambda: head(True), 5),
             "library_logits_gemm_random": (library_logits, 5)}
    out = {"workload": "configs[1] attention fwd+bwd, configs[2] fused-head fwd+bwd and the "
                       "library GEMM h E^T, each back to back; rocm-smi shader clock"}
    for name, (make, batch) in cases.items():
        step = make()
        for _ in range(2 * batch):
            step()
        torch.cuda.synchronize()
        samples, stop = [], threading.Event()

        def sample():
            while not stop.is_set():
                mhz = read_sclk_mhz()
                if mhz is not None:
                    samples.append(mhz)
                time.sleep(0.1)

        th = threading.Thread(target=sample)
        th.start()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            for _ in range(batch):
                step()
            n += batch
            torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / n
        stop.set()
        th.join()
        tail = samples[len(samples) // 2:]  # after the clock has settled
        out[name] = {"ms_per_step": round(dt * 1e3, 4),
                     "sclk_mhz": round(sum(tail) / len(tail), 1) if tail else None,
                     "samples": len(samples)}
        print(json.dumps({name: out[name]}), flush=True)
        del step
        torch.cuda.empty_cache()
    return out


def bench_newton_schulz(steps, warmup, dev):
    """Muon's Newton-Schulz at the 350M model's shapes: the 96 [1024, 1024]
    and 72 [1024, 2688] matrices of one training step (optimizers.py:27-65,
    5 quintic and 2 refinement steps, bf16 products). `iteration_ms` is the
    products alone (both batches in lockstep, one grouped launch per
    product); `ms` is newton_schulz_many end to end (float32 in, the
    normalisation, float32 out). FLOPs count full products (28 m^2 n + 10 m^3
    per matrix), though the symmetric ones form only their upper triangle."""
    import torch
    from algebraic_amd import optimizers as O
    gen = torch.Generator(device=dev).manual_seed(4)
    Gs = [torch.randn((96, 1024, 1024), device=dev, generator=gen),
          torch.randn((72, 1024, 2688), device=dev, generator=gen)]
    Xs = []
    for G in Gs:
        X = torch.empty(G.shape, dtype=torch.bfloat16, device=dev)
        O._normalize_into(G, X, 1e-7)
        Xs.append(X)
    work = [X.clone() for X in Xs]

    def iteration():
        for w, X in zip(work, Xs):
            w.copy_(X)
        O._ns_iterate_many(work, 5)

    def copies():
        for w, X in zip(work, Xs):
            w.copy_(X)

    it_s = time_steps(iteration, steps, warmup)
    copy_s = time_steps(copies, steps, warmup, settle_s=0.0)
    full_s = time_steps(lambda: O.newton_schulz_many(Gs), steps, warmup, settle_s=0.0)
    flops = sum(G.shape[0] * (28 * G.shape[1] ** 2 * G.shape[2] + 10 * G.shape[1] ** 3)
                for G in Gs)
    it_ms = (it_s - copy_s) * 1e3
    return {"workload": "Muon Newton-Schulz, 96 x [1024,1024] + 72 x [1024,2688], bf16, 5+2 steps",
            "iteration_ms": it_ms, "ms": full_s * 1e3,
            "iteration_tflops": flops / it_ms / 1e9,
            "iteration_frac": flops / it_ms / 1e9 / PEAK_BF16_TFLOPS}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true", help="skip the head/QK-norm lines")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--head-only", action="store_true",
                    help="time only the fused head (configs[2]) and print its line (for profiling)")
    ap.add_argument("--model-only", action="store_true",
                    help="print only the 350M model lines (algebraic and standard)")
    ap.add_argument("--elementwise-only", action="store_true",
                    help="print only the rms_norm / alu_glu line")
    ap.add_argument("--clock", action="store_true",
                    help="print only the shader-clock line (attention step on random vs zero "
                         "inputs, rocm-smi sampling)")
    ap.add_argument("--ns-only", action="store_true",
                    help="print only the Newton-Schulz line (Muon at the 350M model's shapes)")
    ap.add_argument("--once", choices=("attn", "attn16", "attn_harness", "head", "qknorm"),
                    help="run three untimed steps of one workload and exit, printing nothing "
                         "else: the command for rocprofv3 counter passes (configs[1] attention, "
                         "configs[3] attention, the reference harness's four attention "
                         "variants, configs[2] head, configs[3] QK-norm)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one plain 256 MiB device copy (scale reference for the "
                         "FETCH_SIZE/WRITE_SIZE counters of a rocprofv3 --pmc run)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: every box in this build has one MI355X and the hot "
              "path is sharded by (b, h) heads with no exchange; run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from algebraic_amd import _lib
    _lib.load()
    dev = "cuda:0"
    B, H, T, D = 8, 12, 2048, 64
    if args.calibrate_copy:
        calibrate_copy(dev)
    if args.once:
        run_once(args.once, dev)
        return
    if args.head_only:
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v)
                          for k, v in bench_head(args.steps, args.warmup, dev).items()}),
              flush=True)
        return
    if args.model_only:
        for preset, remat, opt in (("algebraic", False, False), ("standard", False, False),
                                   ("algebraic", True, False), ("standard", True, False),
                                   ("algebraic", False, True)):
            print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v)
                              for k, v in bench_model(preset, args.steps, args.warmup, dev,
                                                      remat=remat, optimizer=opt).items()}),
                  flush=True)
        return
    if args.elementwise_only:
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v)
                          for k, v in bench_elementwise(args.steps, args.warmup, dev).items()}),
              flush=True)
        return
    if args.clock:
        print(json.dumps(bench_clock(dev)), flush=True)
        return
    if args.ns_only:
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v)
                          for k, v in bench_newton_schulz(args.steps, args.warmup, dev).items()}),
              flush=True)
        return
    torch.cuda.synchronize()
    a = bench_attention(B, H, T, D, args.steps, args.warmup, dev)
    bwd_achieved = a["bwd_flops"] / (a["bwd_kernel_ms"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(a["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(a["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "asinh-power causal flash attention fwd+bwd (configs[1])",
                   "batch": B, "heads": H, "seq_len": T, "head_dim": D, "n": 16, "c": 8.0,
                   "range_guard": True, "sink": None, "qk_norm_inputs": True},
        "roofline": {"bound": "mfma", "kernel": "attention backward (bwd_mfma_kernel)",
                     "achieved": round(bwd_achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(bwd_achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": bwd_counters().get("bytes_per_launch"),
                     "mfma_busy": bwd_counters().get("mfma_busy"),
                     "valu_busy": bwd_counters().get("valu_busy"),
                     # traffic / mfma_busy / valu_busy are not measured by this
                     # run: they are read from the committed counter summary
                     "counters_from": ({"file": "profiles/attn_bwd_traffic.json",
                                        "kernel": bwd_counters().get("kernel"),
                                        "measured_in_this_run": False}
                                       if bwd_counters() else None),
                     "flops_per_launch": a["bwd_flops"],
                     "avg_launch_ms": round(a["bwd_kernel_ms"], 4)},
        "step_frac_of_peak": round(a["tflops"] / PEAK_BF16_TFLOPS, 4),
        "kernels": {
            "attn_fwd": {"avg_launch_ms": round(a["fwd_kernel_ms"], 4),
                         "tflops": round(a["fwd_flops"] / a["fwd_kernel_ms"] / 1e9, 2)},
            "attn_bwd": {"avg_launch_ms": round(a["bwd_kernel_ms"], 4),
                         "tflops": round(bwd_achieved, 2)},
        },
    }
    if not args.no_secondary:
        a16 = bench_attention(8, 16, T, D, max(5, args.steps // 2), 2, dev)
        asm = bench_attention(B, H, T, D, max(5, args.steps // 2), 2, dev, kind="softmax")
        harness = bench_harness_variants(max(5, args.steps // 2), 2, dev)
        # The memory-bound lines run before the head, whose step and library
        # comparison allocate ~5 GB (the 1.65 GB dz among them).
        qk = bench_qknorm(20, 3, dev)
        ew = bench_elementwise(20, 3, dev)
        line["secondary"] = {
            "attn_h16": {"workload": "configs[3] attention B=8,H=16,T=2048,D=64",
                         "ms_per_step": round(a16["ms_per_step"], 4),
                         "tflops": round(a16["tflops"], 2),
                         "frac": round(a16["tflops"] / PEAK_BF16_TFLOPS, 4)},
            "attn_softmax": {"workload": "softmax comparison arm at configs[1] (kind='softmax', "
                                         "bench_attention.py:75-76)",
                             "ms_per_step": round(asm["ms_per_step"], 4),
                             "tflops": round(asm["tflops"], 2),
                             "frac": round(asm["tflops"] / PEAK_BF16_TFLOPS, 4)},
            "attn_harness_variants": harness,
            "fused_head": {k: (round(v, 4) if isinstance(v, float) else v)
                           for k, v in bench_head(5, 2, dev).items()},
            # bench_head.py:48-55: alg_ce at the harness's defaults (n=16,
            # c=16), and the cross entropy, at configs[2]
            "fused_head_alg_ce_n16_c16": {
                k: (round(v, 4) if isinstance(v, float) else v)
                for k, v in bench_head(5, 2, dev, kind="alg_ce", n=16, c=16.0,
                                       library=False).items()},
            "fused_head_ce": {k: (round(v, 4) if isinstance(v, float) else v)
                              for k, v in bench_head(5, 2, dev, kind="ce", n=16, c=16.0,
                                                     library=False).items()},
            "qknorm": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in qk.items()},
            "elementwise": {k: (round(v, 4) if isinstance(v, float) else v)
                            for k, v in ew.items()},
            "newton_schulz": {k: (round(v, 4) if isinstance(v, float) else v)
                              for k, v in bench_newton_schulz(5, 2, dev).items()},
        }
        for preset, remat, opt in (("algebraic", False, False), ("standard", False, False),
                                   ("algebraic", True, False), ("algebraic", False, True)):
            key = f"model_350m_{preset}{'_remat' if remat else ''}{'_train' if opt else ''}"
            line["secondary"][key] = {
                k: (round(v, 4) if isinstance(v, float) else v)
                for k, v in bench_model(preset, 5, 2, dev, remat=remat, optimizer=opt).items()}
    if not args.no_cpu:
        line["cpu_baseline"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                for k, v in cpu_baseline(B, H, T, D).items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
