#!/usr/bin/env python3
"""Benchmark of the MI355X log-linear attention hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step = one log-linear Mamba-2 chunkwise forward (``hattention_kernel``,
HStruct.MAMBA2, the fused HIP kernels) over one batch of synthetic inputs at
the BASELINE north-star shape B=4, T=16384, H=16, dk=dv=64, L=15, bf16
q/k/v/lambda, fp32 g, inputs resident in HBM.  Each step first evicts the
256 MB memory-side cache (a 1 GiB read, outside the timed events), then runs
the forward between HIP events on the launch stream; ``value`` and the
roofline use the median step (cold memory-side cache, median of the reps), the back-to-back (warm)
figures are kept under ``timing``.  Prints one JSON line with the throughput
(tokens/s), the HBM roofline (algorithmic bytes / median forward time), the
other BASELINE configs (C1, C2, C2 bf16x3, C4 forward + backward, the GDN
config 3 forward and forward + backward) with their rooflines, the decode
step, the Mamba-2 layer and a host-CPU baseline (this repo's fp32 torch
restatements of the reference's chunkwise and recurrent algorithms, timed
on bounded samples).

Only one GPU is used: ``--gpus`` above 1 exits with a message.
"""
import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "log-linear-attention_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

# north-star workload
NS = dict(B=4, T=16384, H=16, K=64, V=64, L=15)
HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15    # FLOP/s dense bf16


def make_mamba2_inputs(B, T, H, K, V, L, G=None, seed=1000, dtype=torch.bfloat16,
                       ldtype=None, device="cpu", with_do=False):
    """Seeded synthetic inputs of the BASELINE configs (drawn fp32 on CPU in the
    order q, k, v, A_log, dt-noise, lambda-noise, (dO), then cast / moved).

    A = exp(A_log), A_log ~ U[log 1, log 16] per head; dt = clamp(softplus(N(0,1)
    + b_h), 1e-3, 1e-1) with b_h = softplus^-1(dt0_h), dt0_h = exp(U[log 1e-3,
    log 1e-1]); g = -A * dt (fp32); lambda = softplus(N(0,1)).
    """
    G = G or H
    ldtype = ldtype or dtype
    gen = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, T, G, K, generator=gen)
    k = torch.randn(B, T, G, K, generator=gen)
    v = torch.randn(B, T, H, V, generator=gen)
    A_log = torch.empty(H).uniform_(math.log(1.0), math.log(16.0), generator=gen)
    dt0 = torch.exp(torch.empty(H).uniform_(math.log(1e-3), math.log(1e-1), generator=gen))
    bias = dt0 + torch.log(-torch.expm1(-dt0))                  # softplus^-1
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen) + bias)
    dt = dt.clamp(1e-3, 1e-1)
    g = (-torch.exp(A_log) * dt).float()
    lam = torch.nn.functional.softplus(torch.randn(B, T, H, L, generator=gen))
    out = [q.to(dtype), k.to(dtype), v.to(dtype), g, lam.to(ldtype)]
    if with_do:
        out.append(torch.randn(B, T, H, V, generator=gen).to(dtype))
    return [t.to(device) for t in out]


def make_gdn_inputs(B, T, H, K, V, L, seed=1003, dtype=torch.bfloat16, device="cpu"):
    """Seeded GDN inputs of BASELINE config 3 (drawn fp32 on CPU in the order q, k,
    v, A_log, dt-noise, lambda-noise, beta-noise): q, k l2-normalised N(0,1);
    v ~ N(0,1); beta = sigmoid(N(0,1)); g = -A * dt as in the Mamba-2 configs;
    lambda = softplus(N(0,1))."""
    gen = torch.Generator("cpu").manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=gen), dim=-1)
    v = torch.randn(B, T, H, V, generator=gen)
    A_log = torch.empty(H).uniform_(math.log(1.0), math.log(16.0), generator=gen)
    dt0 = torch.exp(torch.empty(H).uniform_(math.log(1e-3), math.log(1e-1), generator=gen))
    bias = dt0 + torch.log(-torch.expm1(-dt0))
    dt = torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen) + bias)
    dt = dt.clamp(1e-3, 1e-1)
    g = (-torch.exp(A_log) * dt).float()
    lam = torch.nn.functional.softplus(torch.randn(B, T, H, L, generator=gen))
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    out = [q.to(dtype), k.to(dtype), v.to(dtype), beta.to(dtype), g, lam.to(dtype)]
    return [t.to(device) for t in out]


def fwd_bytes(B, T, H, K, V, L, es=2, es_l=2, G=None):
    """Algorithmic HBM bytes of one forward: read q, k, v, g, lambda, write o."""
    G = G or H
    return B * T * (2 * G * K * es + H * V * es + H * V * es + H * 4 + H * L * es_l)


def fwd_flops(B, T, H, K, V):
    nlev = math.ceil(math.log2(T // 64)) if T > 64 else 0
    return B * H * (2 * T * 64 * (K + V) + 2 * T * K * V + T * K * V * nlev)


def bwd_bytes(B, T, H, K, V, L, es=2, es_l=2):
    """Algorithmic HBM bytes of one backward: read q, k, v, g, lambda, dO,
    write dq, dk, dv (input dtypes), dg and dlambda (fp32)."""
    return B * T * H * (2 * K * es + V * es + 4 + L * es_l + V * es      # inputs + dO
                        + 2 * K * es + V * es + 4 + L * 4)              # gradients


def bwd_flops(B, T, H, K, V):
    nlev = math.ceil(math.log2(T // 64)) if T > 64 else 0
    return B * H * (2 * T * 64 * (3 * K + 2 * V) + 6 * T * K * V + 2 * T * K * V * nlev)


def gdn_fwd_flops(B, T, H, K, V):
    """Algorithmic FLOPs of the GDN forward per (b, h) (KK^T, w, intra QK^T, the
    two q_new products, u, A V, A Aw, the triangular solve, and nlev delta-rule
    recurrences plus level reads)."""
    BT = 64
    nlev = math.ceil(math.log2(T // BT)) if T > BT else 0
    return B * H * (2 * T * BT * (5 * K + 2 * V + BT) + (2 / 3) * BT * BT * T
                    + 5 * T * K * V * nlev)


def measured_traffic(path=os.path.join(ROOT, "profiles", "mamba2_fwd_ns_traffic.txt")):
    """HBM bytes per forward launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (line 'traffic_bytes: N'), or None."""
    try:
        for line in open(path):
            if line.startswith("traffic_bytes:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _median(xs):
    xs = sorted(xs)
    n = len(xs)
    return xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])


class Evictor:
    """A 1 GiB buffer read before each timed rep: four times the 256 MB
    memory-side cache (MALL), so no line of the previous rep survives.  A read
    (a reduction into one value) leaves only clean lines behind; a write fill
    would leave 256 MB of dirty lines whose write-back then lands inside the
    timed rep."""

    def __init__(self, dev):
        self.buf = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=dev)
        self.out = torch.empty((), dtype=torch.float32, device=dev)

    def __call__(self):
        torch.sum(self.buf, (0,), out=self.out)


def time_cold(fn, reps, stream, evict):
    """Cold-cache protocol: before each rep the memory-side cache is
    evicted (outside the events); each rep is bracketed by HIP events on the
    launch stream.  Returns the per-rep event times in seconds."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    torch.cuda.synchronize()
    for a, b in ev:
        evict()
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) / 1e3 for a, b in ev]


def _time_region(fn, n, stream):
    """Run fn n times; return (wall seconds per call, HIP-event seconds per call on
    the launch stream)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(n):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / n, e0.elapsed_time(e1) / 1e3 / n


def decode_bench(dev, stream, n_steps, warmup):
    """Decode steps (hattention_step: cascade, gate, insert and output in one
    launch) from an empty HState: Mamba-2 at the north-star state shape and
    GDN at the config-3 state shape, per-token inputs contiguous [B, H, D].
    The HBM bytes per step are the state's read and write (the per-token
    operands are < 0.1 percent)."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_step
    from hattention.recurrent import HState
    res = {}
    for name, hs, (B, H, K, V, L) in (("mamba2", HStruct.MAMBA2, (4, 16, 64, 64, 16)),
                                      ("gdn", HStruct.GDELTA, (4, 16, 128, 128, 14))):
        T = n_steps + warmup
        if hs == HStruct.MAMBA2:
            q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, seed=1004, device=dev)
            b, scale, norm = None, None, False
        else:
            q, k, v, b, g, l = make_gdn_inputs(B, T, H, K, V, L, seed=1005, device=dev)
            scale, norm = K ** -0.5, True
        # token-major copies split into per-token views up front, so a step's
        # host time is hattention_step's own, not the harness's tensor indexing
        tm = lambda x: list(x.transpose(0, 1).contiguous().unbind(0)) if x is not None else None
        q, k, v, b, g, l = (tm(x) for x in (q, k, v, b, g, l))
        S = HState(2, HType.WEAK, hs, (B, H, K, V, L), torch.float32, dev)
        it = iter(range(T))

        def step():
            t = next(it)
            return hattention_step(S, q[t], k[t], v[t], b[t] if b is not None else None, g[t],
                                   l[t], scale, 2, HType.WEAK, hs, use_qk_l2norm_in_kernel=norm)

        for _ in range(warmup):
            step()
        wall, ev = _time_region(step, n_steps, stream)
        nbytes = 2 * B * H * K * V * L * 4
        res[name] = {"state": {"batch": B, "heads": H, "dk": K, "dv": V, "levels": L,
                               "dtype_state": "fp32", "dtype_qkv": "bf16"},
                     "us_per_step": wall * 1e6, "steps": n_steps,
                     "roofline": {"bound": "hbm", "achieved": nbytes / ev / 1e9,
                                  "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                                  "frac": nbytes / ev / HBM_PEAK, "algorithmic_bytes": nbytes,
                                  "avg_step_us": ev * 1e6}}
        del q, k, v, b, g, l, S
    return res


def layer_bench(dev, stream, n_steps, warmup):
    """The Mamba-2 layer scan of hmamba_chunk_scan_combined at the north-star
    shape (x [4, 16384, 16, 64] bf16, B = C [4, 16384, 16, 64] bf16, dl bf16 with
    15 levels, positive lambda, D and dt_bias): the fused HIP pre- / post-
    processing around the scan, against the same scan kernels wrapped in the
    reference's torch expressions (mamba_apis.py:346-403), forward and
    forward + backward.  HBM bytes of the fused forward: x, B, C, dt, dl read
    and y written once by the kernels plus the v / g / lambda round trip."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_kernel
    from hattention.mamba_apis import hmamba_chunk_scan_combined
    B, T, H, P, N, L = NS["B"], NS["T"], NS["H"], NS["V"], NS["K"], NS["L"]
    gen = torch.Generator("cpu").manual_seed(1006)
    x = torch.randn(B, T, H, P, generator=gen).bfloat16().to(dev)
    dt = (torch.randn(B, T, H, generator=gen) * 0.5 - 2.5).to(dev)
    A = -torch.exp(torch.rand(H, generator=gen)).to(dev)
    Bm = torch.randn(B, T, H, N, generator=gen).bfloat16().to(dev)
    Cm = torch.randn(B, T, H, N, generator=gen).bfloat16().to(dev)
    dl = torch.randn(B, T, H, L, generator=gen).bfloat16().to(dev)
    Lp = (torch.randn(H, L, generator=gen) * 0.5).to(dev)
    D = torch.randn(H, generator=gen).to(dev)
    bias = (torch.randn(H, generator=gen) * 0.1).to(dev)
    kw = dict(lambda_mode="positive", lambda_level_max=L, lambda_level_base=2,
              lambda_htype=HType.WEAK, lambda_hstruct=HStruct.MAMBA2, lambda_level_fixed=True)

    def fused(*a):
        return hmamba_chunk_scan_combined(*a[:7], 64, D=a[7], dt_bias=a[8], dt_softplus=True,
                                          **kw)[0]

    def chain(*a):
        d = torch.nn.functional.softplus(a[1] + a[8][None, None])
        lam = torch.nn.functional.softplus(a[6][None, None] * a[5])
        y = hattention_kernel(a[4], a[3], a[0] * d[..., None], None, a[2][None, None] * d, lam,
                              None, False, 2, HType.WEAK, HStruct.MAMBA2)
        return y + a[0] * a[7][None, None, :, None]

    base = (x, dt, A, Bm, Cm, dl, Lp, D, bias)
    dy = torch.randn(B, T, H, P, device=dev)
    res = {}
    for name, fn in (("fused", fused), ("torch_chain", chain)):
        with torch.no_grad():
            for _ in range(warmup):
                fn(*base)
            wall_f, _ = _time_region(lambda: fn(*base), n_steps, stream)
        leaves = [t.detach().clone().requires_grad_(True) for t in base]

        def fb():
            for t in leaves:
                t.grad = None
            fn(*leaves).backward(dy)

        for _ in range(max(1, warmup)):
            fb()
        wall_fb, _ = _time_region(fb, n_steps, stream)
        res[name] = {"fwd_tokens_per_s": B * T / wall_f, "fwd_ms": wall_f * 1e3,
                     "fwd_bwd_tokens_per_s": B * T / wall_fb, "fwd_bwd_ms": wall_fb * 1e3}
        del leaves
    res["shape"] = {"batch": B, "seq_len": T, "heads": H, "headdim": P, "dstate": N,
                    "levels": L, "lambda_mode": "positive", "dtype_x_bc_dl": "bf16"}
    del base, dy, x, dt, Bm, Cm, dl
    res["split_conv1d"] = split_layer_bench(dev, stream, n_steps, warmup)
    return res


def split_layer_bench(dev, stream, n_steps, warmup):
    """hmamba_split_conv1d_scan_combined at the north-star scan shape (ngroups 1,
    conv width 4, out-projection 1024 -> 1024, zxbcdtdl bf16, fp32 parameters):
    the HIP conv1d + SiLU and gated RMSNorm kernels around the fused scan,
    against torch's grouped conv1d and the RMSNorm expressions around the same
    scan.  Forward and forward + backward."""
    from hattention.base import HType, HStruct
    from hattention.mamba_apis import hmamba_chunk_scan_combined, hmamba_split_conv1d_scan_combined
    B, T, H, P, N, L, G, W = NS["B"], NS["T"], NS["H"], NS["V"], NS["K"], NS["L"], 1, 4
    dim = H * P
    width = 2 * dim + 2 * G * N + H + H * L
    gen = torch.Generator("cpu").manual_seed(1007)
    zx = torch.randn(B, T, width, generator=gen)
    zx[..., 2 * dim + 2 * G * N:2 * dim + 2 * G * N + H] -= 2.5
    zx = zx.bfloat16().to(dev)
    prm = [t.to(dev) for t in (torch.randn(dim + 2 * G * N, W, generator=gen) * 0.5,
                               torch.randn(dim + 2 * G * N, generator=gen) * 0.1,
                               torch.randn(H, generator=gen) * 0.1,
                               -torch.exp(torch.rand(H, generator=gen)),
                               torch.randn(H, L, generator=gen) * 0.5, torch.randn(H, generator=gen),
                               1 + 0.1 * torch.randn(dim, generator=gen),
                               torch.randn(dim, dim, generator=gen) / dim ** 0.5,
                               torch.randn(dim, generator=gen) * 0.1)]
    kw = dict(lambda_mode="positive", lambda_level_max=L, lambda_level_base=2,
              lambda_htype=HType.WEAK, lambda_hstruct=HStruct.MAMBA2, lambda_level_fixed=True)

    def fused(z, cw, cb, db, A, Lp, D, rw, ow, ob):
        return hmamba_split_conv1d_scan_combined(
            z, cw, cb, db, A, Lp, D, 64, rmsnorm_weight=rw, rmsnorm_eps=1e-6, outproj_weight=ow,
            outproj_bias=ob, headdim=P, ngroups=G, norm_before_gate=False, **kw)

    def chain(z, cw, cb, db, A, Lp, D, rw, ow, ob):
        zz, xBC, dt, dl = torch.split(z, [dim, dim + 2 * G * N, H, H * L], dim=-1)
        xBC = torch.nn.functional.conv1d(torch.nn.functional.pad(xBC.transpose(1, 2), (W - 1, 0)),
                                         cw[:, None, :].to(z.dtype), cb.to(z.dtype),
                                         groups=dim + 2 * G * N)
        xBC = torch.nn.functional.silu(xBC).transpose(1, 2)
        x, Bm, Cm = torch.split(xBC, [dim, G * N, G * N], dim=-1)
        y, _ = hmamba_chunk_scan_combined(x.reshape(B, T, H, P), dt, A, Bm.reshape(B, T, G, N),
                                          Cm.reshape(B, T, G, N), dl.reshape(B, T, H, L), Lp, 64,
                                          D=D, dt_bias=db, dt_softplus=True, **kw)
        u = y.reshape(B, T, dim) * torch.nn.functional.silu(zz)
        u = u * torch.rsqrt((u * u).mean(-1, keepdim=True) + 1e-6) * rw
        return torch.nn.functional.linear(u, ow, ob)

    res = {}
    for name, fn in (("fused", fused), ("torch_conv_norm", chain)):
        with torch.no_grad():
            for _ in range(warmup):
                fn(zx, *prm)
            wall_f, _ = _time_region(lambda: fn(zx, *prm), n_steps, stream)
        leaves = [zx.detach().clone().requires_grad_(True)] + \
            [t.detach().clone().requires_grad_(True) for t in prm]

        def fb():
            for t in leaves:
                t.grad = None
            fn(*leaves).sum().backward()

        for _ in range(max(1, warmup)):
            fb()
        wall_fb, _ = _time_region(fb, n_steps, stream)
        res[name] = {"fwd_tokens_per_s": B * T / wall_f, "fwd_ms": wall_f * 1e3,
                     "fwd_bwd_tokens_per_s": B * T / wall_fb, "fwd_bwd_ms": wall_fb * 1e3}
        del leaves
    res["shape"] = {"batch": B, "seq_len": T, "d_inner": dim, "heads": H, "headdim": P,
                    "dstate": N, "ngroups": G, "conv_width": W, "levels": L, "d_out": dim}
    return res


def cpu_model():
    """CPU model name of the host (first 'model name' line of /proc/cpuinfo)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _progress(msg):
    """One progress line on stderr (stdout carries only the JSON record)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(seconds_budget=20.0):
    """Host-CPU baselines (the chunkwise and recurrent forms on the host cores), all fp32 torch restatements
    of the reference (the reference itself cannot run on the box):
    * chunkwise: oracle.mamba2.chunked_scan_fwd (the reference's chunkwise
      level-scan algorithm, chunkwise.py:1118-1275) at the full north-star, C1
      and C4 shapes, median of up to 3 runs within the budget each;
    * recurrent: oracle.mamba2.recurrent_fwd (the Fenwick state machine of
      recurrent.py:9-216) on config 0 in full and on a 2048-token prefix of the
      north-star shape (its cost per token does not depend on T at fixed L),
      median of up to 3 runs within 100 s.
    ``value`` is the chunkwise north-star figure (the GPU headline's workload)."""
    from oracle.mamba2 import chunked_scan_fwd, recurrent_fwd
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)

    def run(fn, shape, seed, budget):
        B, T, H, K, V, L = shape
        q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, seed=seed, dtype=torch.float32)
        times = []
        t_start = time.perf_counter()
        while len(times) < 3 and (time.perf_counter() - t_start) < budget:
            t0 = time.perf_counter()
            fn(q, k, v, g, l)
            times.append(time.perf_counter() - t0)
        t = _median(times)
        _progress(f"cpu {getattr(fn, '__name__', 'fn')} {shape}: {t:.2f} s x {len(times)}")
        return {"tokens_per_s": B * T / t, "seconds": t, "runs": len(times),
                "shape": dict(zip(("batch", "seq_len", "heads", "dk", "dv", "levels"), shape))}

    chunk = lambda *a: chunked_scan_fwd(*a, chunk_size=64)
    res = {
        "chunkwise_ns": run(chunk, (4, 16384, 16, 64, 64, 15), 1000, seconds_budget),
        "chunkwise_c1": run(chunk, (8, 4096, 16, 64, 64, 13), 1001, seconds_budget / 2),
        "chunkwise_c4": run(chunk, (8, 8192, 24, 64, 64, 14), 1004, seconds_budget / 2),
        "recurrent_c0": run(recurrent_fwd, (2, 1024, 4, 64, 64, 11), 1000, 1.0),
        # median of up to 3 runs of a 2048-token prefix (one run takes ~40-60 s)
        "recurrent_ns_prefix2048": run(recurrent_fwd, (4, 2048, 16, 64, 64, 15), 1000, 100.0),
    }
    t = res["chunkwise_ns"]
    return {
        "value": t["tokens_per_s"],
        "unit": "tokens/s",
        "cores": n,
        "kind": "port",
        "cpu": cpu_model(),
        "sample": (f"fp32 torch chunked level-scan restatement (oracle/mamba2.py "
                   f"chunked_scan_fwd) on the full north-star workload B=4 T=16384 H=16 "
                   f"dk=dv=64 L=15, median of {t['runs']} runs ({t['seconds']:.2f}s each), "
                   f"{n} threads on {cpu_model()}; more shapes and the recurrent form in "
                   f"'detail'"),
        "detail": res,
    }


def mamba2_fwd_record(name, shape, dtype, dev, stream, evict, reps, warmup, backward=False,
                      strong=False):
    """Cold-cache median (memory-side cache evicted before each rep) of one Mamba-2 chunkwise forward
    (or forward + backward through HAttentionFunction) at one BASELINE config,
    with its roofline: HBM-bound by algorithmic bytes (q, k, v, g, lambda read and o written once).
    ``strong``: the strong hierarchy (HType.STRONG) on the same inputs."""
    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_kernel
    ht = HType.STRONG if strong else HType.WEAK
    B, T, H, K, V, L = shape
    es = 4 if dtype == torch.float32 else 2
    q, k, v, g, l, do = make_mamba2_inputs(B, T, H, K, V, L, seed=1000, dtype=dtype, device=dev,
                                           with_do=True)
    if backward:
        leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v, g, l)]

        def fn():
            for x in leaves:
                x.grad = None
            hattention_kernel(leaves[0], leaves[1], leaves[2], None, leaves[3], leaves[4], None,
                              False, 2, ht, HStruct.MAMBA2).backward(do)
    else:
        def fn():
            with torch.no_grad():
                hattention_kernel(q, k, v, None, g, l, None, False, 2, ht, HStruct.MAMBA2)
    for _ in range(warmup):
        fn()
    times = time_cold(fn, reps, stream, evict)
    t = _median(times)
    _progress(f"{name}{' strong' if strong else ''}: {t * 1e6:.1f} us")
    nbytes = fwd_bytes(B, T, H, K, V, L, es=es, es_l=es)
    flops = fwd_flops(B, T, H, K, V)
    if backward:
        nbytes += bwd_bytes(B, T, H, K, V, L, es=es, es_l=es)
        flops += bwd_flops(B, T, H, K, V)
    mfma_equiv = flops * (3 if dtype == torch.float32 else 1)   # bf16x3: three MFMAs a product
    t_roof = max(nbytes / HBM_PEAK, mfma_equiv / MFMA_BF16_PEAK)
    bound = "hbm" if nbytes / HBM_PEAK >= mfma_equiv / MFMA_BF16_PEAK else "mfma"
    del q, k, v, g, l, do
    return {"config": name, "batch": B, "seq_len": T, "heads": H, "dk": K, "dv": V, "levels": L,
            "htype": ht.name,
            "dtype": "fp32 (bf16x3)" if dtype == torch.float32 else "bf16",
            "pass": "fwd+bwd" if backward else "fwd",
            "value": B * T / t, "unit": "tokens/s", "median_us": t * 1e6,
            "reps": reps, "min_us": min(times) * 1e6, "max_us": max(times) * 1e6,
            "roofline": {"bound": bound,
                         "achieved": (nbytes / t / 1e9) if bound == "hbm" else mfma_equiv / t / 1e12,
                         "peak": HBM_PEAK / 1e9 if bound == "hbm" else MFMA_BF16_PEAK / 1e12,
                         "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
                         "frac": t_roof / t, "algorithmic_bytes": nbytes,
                         "algorithmic_flops": flops}}


GDN_C3 = (4, 8192, 16, 128, 128, 14)


def gdn_records(dev, stream, evict, reps, keys=("fwd", "fwd_bwd"), shape=GDN_C3, warmup=5):
    """Cold-cache medians of the log-linear Gated DeltaNet chunkwise forward
    (chunkwise_hgdn.chunkwise_fwd) and forward + backward (chunkwise_fwd_keep /
    chunkwise_bwd with the kept workspace, the HAttentionFunction path) at
    BASELINE config 3, MFMA roofline by the algorithmic FLOPs (backward counted
    as twice the forward, the usual convention).  Returns one record per key
    (None for keys not asked for)."""
    from hattention.base import HType
    from hattention.chunkwise_hgdn import (chunkwise_fwd as gdn_fwd, chunkwise_bwd as gdn_bwd,
                                           chunkwise_fwd_keep as gdn_fwd_keep)
    GB, GT, GH, GK, GV, GL = shape
    gq, gk, gv, gbeta, gg, gl = make_gdn_inputs(GB, GT, GH, GK, GV, GL, device=dev)
    gdo = torch.randn(GB, GT, GH, GV, device=dev, dtype=torch.bfloat16)
    gcfg = {"workload": "log-linear Gated DeltaNet chunkwise path (chunkwise_hgdn, "
                        "BASELINE config 3)",
            "batch": GB, "seq_len": GT, "heads": GH, "dk": GK, "dv": GV, "levels": GL}

    def gdn_step():
        return gdn_fwd(gq, gk, gv, gbeta, gg, gl, False, 2, HType.WEAK, 64, False)

    def gdn_fb_step():
        # as HAttentionFunction: the forward keeps what the backward would recompute
        gc, _, Aw, Au, _, fws = gdn_fwd_keep(gq, gk, gv, gbeta, gg, gl, False, 2, HType.WEAK, 64,
                                             False)
        return gdn_bwd(gq, gk, gv, gbeta, gc, gl, Aw, Au, gdo, False, 2, HType.WEAK, 64,
                       fwd_ws=fws)

    gfl = gdn_fwd_flops(GB, GT, GH, GK, GV)
    out = {}
    for fn, key in ((gdn_step, "fwd"), (gdn_fb_step, "fwd_bwd")):
        if key not in keys:
            out[key] = None
            continue
        for _ in range(warmup):
            fn()
        times = time_cold(fn, reps, stream, evict)
        t_g = _median(times)
        _progress(f"gdn {key}: {t_g * 1e6:.1f} us")
        fl = gfl if key == "fwd" else 3 * gfl
        out[key] = {"value": GB * GT / t_g, "unit": "tokens/s", "median_us": t_g * 1e6,
                    "reps": reps, "config": gcfg,
                    "roofline": {"bound": "mfma", "achieved": fl / t_g / 1e12,
                                 "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                                 "frac": fl / t_g / MFMA_BF16_PEAK, "algorithmic_flops": fl}}
    del gq, gk, gv, gbeta, gg, gl, gdo
    return out["fwd"], out["fwd_bwd"]


NS_SHAPE = (NS["B"], NS["T"], NS["H"], NS["K"], NS["V"], NS["L"])
ONLY_CASES = {
    "ns_fwd": None,      # the headline loop alone (--fwd-only --no-cpu-baseline)
    "ns_fwd_bwd": lambda dev, st, ev, n, w: mamba2_fwd_record(
        "north star fwd+bwd", NS_SHAPE, torch.bfloat16, dev, st, ev, n, w, backward=True),
    "c2_fwd": lambda dev, st, ev, n, w: mamba2_fwd_record(
        "C2", (1, 32768, 32, 64, 128, 16), torch.bfloat16, dev, st, ev, n, w),
    "c2_x3_fwd": lambda dev, st, ev, n, w: mamba2_fwd_record(
        "C2 bf16x3", (1, 32768, 32, 64, 128, 16), torch.float32, dev, st, ev, n, w),
    "c4_fwd_bwd": lambda dev, st, ev, n, w: mamba2_fwd_record(
        "C4 fwd+bwd", (8, 8192, 24, 64, 64, 14), torch.bfloat16, dev, st, ev, n, w,
        backward=True),
    "ns_strong_fwd": lambda dev, st, ev, n, w: mamba2_fwd_record(
        "north star fwd, HType.STRONG", NS_SHAPE, torch.bfloat16, dev, st, ev, n, w, strong=True),
    "ns_strong_fwd_bwd": lambda dev, st, ev, n, w: mamba2_fwd_record(
        "north star fwd+bwd, HType.STRONG", NS_SHAPE, torch.bfloat16, dev, st, ev, n, w,
        backward=True, strong=True),
    "decode": lambda dev, st, ev, n, w: decode_bench(dev, st, max(n, 128), w),
    "gdn_fwd": lambda dev, st, ev, n, w: gdn_records(dev, st, ev, n, keys=("fwd",))[0],
    "gdn_fwd_bwd": lambda dev, st, ev, n, w: gdn_records(dev, st, ev, n, keys=("fwd_bwd",))[1],
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--fwd-only", action="store_true",
                    help="only the north-star forward (no other configs, backward, decode, layer)")
    ap.add_argument("--calib", action="store_true",
                    help="also run a 2 GiB read-only kernel (sum) and a 2 GiB write-only kernel "
                         "(fill), larger than the 256 MB MALL, so a counter run can scale "
                         "FETCH_SIZE / WRITE_SIZE by a known traffic")
    ap.add_argument("--only", choices=sorted(ONLY_CASES),
                    help="time one case alone (cold-cache median over --steps reps) and print "
                         "its record: the driver of the per-kernel profiles")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(every (batch, head) row is independent, so rows would shard over GPUs "
              "without communication)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)

    from hattention.base import HType, HStruct
    from hattention.kernel import hattention_kernel

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    if args.only and args.only != "ns_fwd":
        evict = Evictor(dev)
        rec = ONLY_CASES[args.only](dev, stream, evict, args.steps, args.warmup)
        print(json.dumps({"case": args.only, "record": rec}), flush=True)
        return
    if args.only == "ns_fwd":
        args.fwd_only, args.no_cpu_baseline = True, True
    B, T, H, K, V, L = (NS[x] for x in ("B", "T", "H", "K", "V", "L"))
    q, k, v, g, l = make_mamba2_inputs(B, T, H, K, V, L, seed=1000, device=dev)
    evict = Evictor(dev)
    torch.cuda.synchronize()

    def step():
        with torch.no_grad():
            return hattention_kernel(q, k, v, None, g, l, None, False, 2, HType.WEAK,
                                     HStruct.MAMBA2)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    if args.calib:
        src = torch.ones(512 * 1024 * 1024, dtype=torch.float32, device=dev)   # 2 GiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.fill_(0.5)        # writes 2 GiB
            src.sum()             # reads 2 GiB (src last written long before, evicted by dst)
        torch.cuda.synchronize()
        del src, dst

    # headline: K steps, each = evict the memory-side cache (outside the events),
    # then one forward bracketed by HIP events; value = tokens / median forward
    t0 = time.perf_counter()
    cold = time_cold(step, args.steps, stream, evict)
    wall = time.perf_counter() - t0
    t_med = _median(cold)
    # the same forward back to back (warm memory-side cache), as a secondary figure
    warm = time_cold(step, args.steps, stream, lambda: None)
    tokens = B * T
    nbytes = fwd_bytes(B, T, H, K, V, L)
    flops = fwd_flops(B, T, H, K, V)

    records = []
    fb = gdn = gdn_fb = dec = layer = None
    if not args.fwd_only:
        # every secondary record: >= 20 cold reps after >= 5 warm-ups
        reps, wu = max(20, args.steps), max(5, args.warmup)
        # north-star forward + backward, then the other BASELINE configs
        fb = mamba2_fwd_record("north star fwd+bwd", (B, T, H, K, V, L), torch.bfloat16, dev,
                               stream, evict, reps, wu, backward=True)
        for name, shape, dt, bw in (
                ("C1", (8, 4096, 16, 64, 64, 13), torch.bfloat16, False),
                ("C2", (1, 32768, 32, 64, 128, 16), torch.bfloat16, False),
                ("C2 bf16x3", (1, 32768, 32, 64, 128, 16), torch.float32, False),
                ("C4 fwd+bwd", (8, 8192, 24, 64, 64, 14), torch.bfloat16, True)):
            records.append(mamba2_fwd_record(name, shape, dt, dev, stream, evict, reps, wu,
                                             backward=bw))
            torch.cuda.empty_cache()
        # the strong hierarchy (HType.STRONG) at the north-star shape
        for bw in (False, True):
            records.append(mamba2_fwd_record(
                "north star fwd+bwd, HType.STRONG" if bw else "north star fwd, HType.STRONG",
                (B, T, H, K, V, L), torch.bfloat16, dev, stream, evict, reps, wu, backward=bw,
                strong=True))
            torch.cuda.empty_cache()

        # log-linear Gated DeltaNet at BASELINE config 3 (MFMA-bound path)
        gdn, gdn_fb = gdn_records(dev, stream, evict, reps, warmup=wu)
        torch.cuda.empty_cache()
        dec = decode_bench(dev, stream, 128, 8)
        layer = layer_bench(dev, stream, reps, wu)

    out = {
        "metric": "fwd tokens/s @B=4,T=16K,H=16,d=64 bf16; % MFMA/HBM roofline; fwd+bwd tok/s",
        "value": tokens / t_med,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_med * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, softplus lambda, Mamba-2 dt/A decay)",
        "config": {"workload": "log-linear Mamba-2 chunkwise forward (hattention_kernel, "
                               "MAMBA2, WEAK, base 2, chunk 64)",
                   "batch": B, "seq_len": T, "heads": H, "dk": K, "dv": V, "levels": L,
                   "dtype_qkv_lambda": "bf16", "dtype_g": "fp32"},
        "timing": {"protocol": "per step: a 1 GiB read (a reduction) evicts the 256 MB "
                               "memory-side cache (outside the events), then one forward "
                               "between HIP events on the launch stream; value and "
                               "ms_per_step use the median",
                   "cold_median_us": t_med * 1e6, "cold_min_us": min(cold) * 1e6,
                   "cold_max_us": max(cold) * 1e6,
                   "wall_ms_per_step_incl_evict": wall / args.steps * 1e3,
                   "warm_mean_us": sum(warm) / len(warm) * 1e6,
                   "warm_median_us": _median(warm) * 1e6},
        "roofline": {"bound": "hbm", "achieved": nbytes / t_med / 1e9, "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": nbytes / t_med / HBM_PEAK,
                     "traffic": measured_traffic(), "algorithmic_bytes": nbytes,
                     "median_launch_us": t_med * 1e6,
                     "mfma_frac": flops / t_med / MFMA_BF16_PEAK,
                     "warm_frac": nbytes / _median(warm) / HBM_PEAK},
        "fwd_bwd": fb,
        "configs": records,
        "gdn_fwd": gdn,
        "gdn_fwd_bwd": gdn_fb,
        "decode": dec,
        "mamba2_layer": layer,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
