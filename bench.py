"""Benchmark: VisionMamba-2D K=4 train step on one MI355X, plus the selective
scan's fwd+VJP bandwidth, printed as one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--eager]
    python bench.py --scan-driver     (profiling driver, see scan_driver)
    python bench.py --scan-driver-long  (profiling driver, see scan_driver_long)
    python bench.py --scan-driver-small  (profiling driver, see scan_driver_small)

Workload (the step timed): VisionMamba encoder, 2D, K=4 scan directions,
batch 32 of 224x224x1 images ~ N(0,1), patch 16 -> 196 tokens, embed_dim
384 (d_inner 768), d_state 16, depth 6, float32 random-init weights
(Kaiming-uniform projections, S4D-real A, dt bias with softplus(bias) in
[1e-3, 1e-1]); loss = mean of the output features; one step = forward +
loss + backward + AdamW update (the package's one-launch AdamW,
mlx_vision_mamba_amd.optim; --torch-adamw for torch's fused AdamW).  The fp32 projection
GEMMs use the TunableOp picks recorded for this step on MI355X
(mlx_vision_mamba_amd/tuning/, read-only; --default-gemms for the library
defaults).  Inputs are resident on the GPU before the
timed region; W untimed warm-up steps, then exactly K steps between two
device synchronisations.  value = images / second.  The step is captured once
in a HIP graph (after the warm-up) and the K timed steps are K replays of it,
so the host issues one launch per step instead of ~190 kernels through
Python and autograd (whose ~7-10 ms per step otherwise approaches the GPU
time on slower hosts); --eager times the eager loop instead.

roofline: the fused scan backward call (the block's scan VJP with the
softplus and silu-gate gradients inside it; the largest hand-written piece
of the step; its kernels are listed in "kernel"), timed with HIP events on
the stream it runs on, for every launch of an eager timed region of K steps
(after the graph replays; HIP events cannot be timed inside a captured graph
on ROCm, and the replayed kernels are the same); achieved =
algorithmic bytes per launch / mean launch time, against the MI355X HBM3E
peak of 8 TB/s.  traffic = HBM bytes per backward call at this shape from
the rocprofv3 FETCH_SIZE and WRITE_SIZE counters, each scaled by what it
reads for a 512 MiB copy (committed summary in profiles/, made with
`bench.py --scan-driver`), or null when that summary is absent.
valu_busy_per_simd: the share of that kernel's cycles its SIMDs' VALU is
issuing, rocprofv3's VALUBusy counter in the same summary (the backward is
bound by VALU issue, so its HBM fraction follows from its instruction count).
copy_GBps: a plain 512 MiB device-to-device copy on the same GPU, timed with
HIP events (read + written bytes / time): the practical HBM ceiling beside
the 8 TB/s peak.
secondary_flops: the reference formula's work, 37 flop + 3 exp per
(b, t, d, n) element for forward + VJP (mamba_metal_fused.py:33-145), over the
mean fused forward + backward call time, against the 157.3 TFLOP/s fp32
vector peak (reported, not the bound; the scan-only entries carry the same
rate as ref_formula_TFLOPs).

scan: the scan alone (forward + VJP through the C ABI) at B=2, L=196,
D=1536, N=16 fp32 and at B=8, L=16384, D=1536, N=16 with bf16 u/B/C/y/grads,
timed over back-to-back calls with inputs resident in HBM (events split
the stream time between forward and VJP), and as replays of the pair
captured in a HIP graph (graph_fwd_vjp_us: no host time between launches).
The long entry carries each pass's VALUBusy from the committed counter
summary (valu_busy_per_pass): every pass is bound by VALU issue, so the
distance to that bound, not to the HBM peak, is what remains.

cpu_baseline: the oracle's CPU restatement of the reference's sequential
VisionMamba step (materialised discretisation, Python time loop, autograd)
on this host's cores, on a bounded sample (batch 2, one step); beside it
the sequential and chunked scans alone at B=2, L=196, D=1536 and the
sequential scan on a 96-channel slice of B=8, L=16384 (scaled x16 as an upper
bound on the full width).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "selective-scan fwd+VJP GB/s & % HBM peak; VisionMamba-2D train imgs/sec"
HBM_PEAK_GBS = 8000.0
# the reference formula's work per (b, t, d, n) element for forward + VJP
# (mamba_metal_fused.py:33-145), against the MI355X fp32 vector peak
REF_FLOP_PER_ELEMENT = 37
REF_EXP_PER_ELEMENT = 3
FP32_VECTOR_PEAK_TFLOPS = 157.3
BWD_KERNELS = ("mvm_scan_fused_bwd: scan_bwd_kernel<float, float, fused> + reduce_grads_kernel "
               "(one time chunk at this shape, so no aggregate pass)")


def _seeded_model(torch, mvm, device):
    torch.manual_seed(1001)
    model = mvm.VisionMamba(img_size=224, patch_size=16, in_channels=1, embed_dim=384, depth=6,
                            d_state=16, input_dim=2, scan_mode="hip")
    return model.to(device)


TORCH_ADAMW = False  # --torch-adamw


def _adamw(torch, model, capturable):
    """The train step's optimiser (lr 1e-4, otherwise AdamW defaults): the
    package's one-launch AdamW, or torch's fused AdamW with --torch-adamw."""
    if TORCH_ADAMW:
        return torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True, capturable=capturable)
    from mlx_vision_mamba_amd.optim import AdamW
    return AdamW(model.parameters(), lr=1e-4)


def bench_step(torch, mvm, scan, steps, warmup, device, graph=True):
    """Time `steps` train steps after `warmup` untimed ones.

    graph=True: the step (forward, loss, backward, AdamW) is captured once in
    a HIP graph and the timed region is `steps` replays of it.  ROCm cannot
    time events inside a captured graph, so a second timed region follows:
    `steps` eager steps of the same model, with a HIP event pair around
    every scan launch (the launch records).  graph=False, or a capture that
    the runtime refuses: the eager region only.  Returns {"elapsed",
    "issued"} of the value region, the eager region's {"elapsed", "issued"},
    the launch records and the mode that was timed."""
    model = _seeded_model(torch, mvm, device)
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(32, 224, 224, 1, generator=gen).to(device)
    # the captured step needs a capturable optimizer (its step count lives on
    # the device); the eager region uses the plain fused AdamW, whose host
    # path is the cheaper one
    opt = _adamw(torch, model, capturable=graph)
    opt_eager = _adamw(torch, model, capturable=False) if graph else opt

    def step(o=opt):
        o.zero_grad(set_to_none=True)
        loss = model(x).mean()
        loss.backward()
        o.step()
        return loss

    def eager_region():
        records = []
        for _ in range(3 if graph else 0):  # the eager optimizer's first steps
            step(opt_eager)
        torch.cuda.synchronize()
        scan.set_scan_timing(records)
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step(opt_eager)
        issued = time.perf_counter() - t0  # host time to issue the K steps
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        scan.set_scan_timing(None)
        if not math.isfinite(float(loss.detach())):
            raise RuntimeError("non-finite loss")
        return {"elapsed": elapsed, "issued": issued}, records

    def graph_region():
        # warm-up on a side stream (as capture requires); the first forward
        # also lays the direction parameters out in their stacked buffers
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(max(warmup, 3)):
                step()
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize()
        opt.zero_grad(set_to_none=True)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            gloss = model(x).mean()
            gloss.backward()
            opt.step()
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        issued = time.perf_counter() - t0
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        # the loss as a number: the tensor's autograd history would keep the
        # capture stream's gradient-accumulation nodes alive into the eager
        # region
        return {"elapsed": elapsed, "issued": issued}, float(gloss.detach())

    mode = "graph" if graph else "eager"
    if graph:
        try:
            value_region, gloss = graph_region()
            if not math.isfinite(gloss):
                raise FloatingPointError("non-finite loss in the captured step")
        except RuntimeError as err:  # capture refused: time the eager loop
            print(f"bench.py: HIP graph capture failed ({err}); timing the eager loop",
                  file=sys.stderr, flush=True)
            torch.cuda.synchronize()
            mode, graph = "eager (graph capture failed)", False
    if not graph:
        for _ in range(warmup):
            step(opt_eager)
        region, records = eager_region()
        value_region = region
    else:
        region, records = eager_region()
    per = {"fwd": [], "bwd": []}
    for kind, e0, e1, nbytes in records:
        per[kind].append((e0.elapsed_time(e1) * 1e-3, nbytes))
    return value_region, region, per, mode


ENCODERS = {
    # name: (input shape, model kwargs); seeds 2 / 1002 and 3 / 1003 (inputs / weights)
    "3d_K6_B4_128cube": ((4, 128, 128, 128, 1),
                         dict(img_size=128, patch_size=8, input_dim=3), 2),
    "4d_K8_B2_T8_64cube": ((2, 8, 64, 64, 64, 1),
                           dict(img_size=64, patch_size=16, input_dim=4, num_temporal_frames=8,
                                temporal_patch_size=1), 3),
}


def bench_encoder(torch, mvm, scan, name, steps, warmup, device):
    """Train step of the 3D (K=6) or 4D (K=8) VisionMamba encoder
    (vision_mamba.py:156-171): E=384, d_state 16, depth 6, float32,
    synthetic N(0,1) volumes, loss = mean of the output features, AdamW.
    Timed as `steps` replays of the captured step (ms/step, volumes/s), and
    the scan's share from HIP events around every fused scan call of
    `steps` eager steps."""
    shape, kw, seed = ENCODERS[name]
    torch.manual_seed(1000 + seed)
    model = mvm.VisionMamba(in_channels=1, embed_dim=384, depth=6, d_state=16, scan_mode="hip",
                            **kw).to(device)
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(device)
    opt = _adamw(torch, model, capturable=True)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(max(warmup, 3)):
            opt.zero_grad(set_to_none=True)
            model(x).mean().backward()
            opt.step()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    opt.zero_grad(set_to_none=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        model(x).mean().backward()
        opt.step()
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    del g
    # eager steps with every scan launch timed on its stream
    opt_e = _adamw(torch, model, capturable=False)
    for _ in range(2):
        opt_e.zero_grad(set_to_none=True)
        model(x).mean().backward()
        opt_e.step()
    torch.cuda.synchronize()
    records = []
    scan.set_scan_timing(records)
    t1 = time.perf_counter()
    for _ in range(steps):
        opt_e.zero_grad(set_to_none=True)
        loss = model(x).mean()
        loss.backward()
        opt_e.step()
    torch.cuda.synchronize()
    eager = time.perf_counter() - t1
    scan.set_scan_timing(None)
    if not math.isfinite(float(loss.detach())):
        raise RuntimeError(f"{name}: non-finite loss")
    t_f = sum(e0.elapsed_time(e1) for k, e0, e1, _ in records if k == "fwd") * 1e-3 / steps
    t_b = sum(e0.elapsed_time(e1) for k, e0, e1, _ in records if k == "bwd") * 1e-3 / steps
    b_f = sum(nb for k, _, _, nb in records if k == "fwd") / steps
    b_b = sum(nb for k, _, _, nb in records if k == "bwd") / steps
    ms = elapsed / steps * 1e3
    L = model.num_patches
    return {"workload": f"VisionMamba {kw['input_dim']}D K={model.num_directions} train step "
                        f"(fwd + mean loss + bwd + AdamW)",
            "input": "x".join(str(v) for v in shape), "seq_len": L, "directions": model.num_directions,
            "embed_dim": 384, "depth": 6, "steps": steps, "ms_per_step": round(ms, 3),
            "samples_per_s": round(shape[0] / (ms * 1e-3), 2),
            "eager_ms_per_step": round(eager / steps * 1e3, 3),
            "scan_fwd_ms_per_step": round(t_f * 1e3, 3), "scan_bwd_ms_per_step": round(t_b * 1e3, 3),
            "scan_share_of_eager_step": round((t_f + t_b) / (eager / steps), 3),
            "scan_GBps": round((b_f + b_b) / (t_f + t_b) / 1e9, 1),
            "scan_chunk_len": int(scan.chunk_len_for(shape[0] * model.num_directions, L, 768))}


def copy_bandwidth(torch, device, iters=20):
    """Measured HBM bandwidth of a plain 512 MiB device-to-device copy
    (torch's copy kernel: 512 MiB read + 512 MiB written per copy), timed
    with HIP events: the practical ceiling beside the 8 TB/s peak."""
    n = 512 * 1024 * 1024 // 4
    src = torch.ones(n, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    seconds = e0.elapsed_time(e1) * 1e-3 / iters
    return round(2 * n * 4 / seconds / 1e9, 1)


def secondary_flops(elements, seconds):
    """The reference formula's work (REF_FLOP_PER_ELEMENT flop and
    REF_EXP_PER_ELEMENT exp per (b, t, d, n), forward + VJP) over a measured
    fwd + VJP time, against the fp32 vector peak."""
    tflops = REF_FLOP_PER_ELEMENT * elements / seconds / 1e12
    return {"flop_per_element": REF_FLOP_PER_ELEMENT, "exp_per_element": REF_EXP_PER_ELEMENT,
            "elements": elements, "fwd_plus_vjp_us": round(seconds * 1e6, 2),
            "achieved_TFLOPs": round(tflops, 2), "peak_TFLOPs": FP32_VECTOR_PEAK_TFLOPS,
            "frac": round(tflops / FP32_VECTOR_PEAK_TFLOPS, 4)}


def bench_scan(torch, scan, bsz, L, D, N, dtype, iters, device):
    from mlx_vision_mamba_amd import synthetic as scan_inputs
    u, dl, A, Bm, Cm, Dv, g = [t.to(device) for t in scan_inputs.make(bsz, L, D, N, seed=0,
                                                                         dtype=dtype)]
    args = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
            Dv.unsqueeze(0))
    g4 = g.unsqueeze(2)
    for _ in range(3):
        y, ck = scan.scan_forward(*args, save_ckpt=True)
        scan.scan_backward(*args, g4, ckpt=ck)
    torch.cuda.synchronize()
    # back-to-back calls (no synchronisation inside the timed loop): events
    # before each forward and each VJP split the stream time between them
    ev_f = [torch.cuda.Event(enable_timing=True) for _ in range(iters + 1)]
    ev_b = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        ev_f[i].record()
        y, ck = scan.scan_forward(*args, save_ckpt=True)
        ev_b[i].record()
        scan.scan_backward(*args, g4, ckpt=ck)
    ev_f[iters].record()
    torch.cuda.synchronize()
    tf = sum(ev_f[i].elapsed_time(ev_b[i]) for i in range(iters)) * 1e-3 / iters
    tb = sum(ev_b[i].elapsed_time(ev_f[i + 1]) for i in range(iters)) * 1e-3 / iters
    size = 2 if dtype == torch.bfloat16 else 4
    bf, bb = scan.algorithmic_bytes(bsz, L, D, N, size, size)
    total = tf + tb
    out = {
        "shape": f"B={bsz} L={L} D={D} N={N} {'bf16' if size == 2 else 'fp32'}",
        "fwd_us": round(tf * 1e6, 2), "vjp_us": round(tb * 1e6, 2),
        "algorithmic_bytes": bf + bb,
        "GBps": round((bf + bb) / total / 1e9, 1),
        "pct_hbm_peak": round((bf + bb) / total / 1e9 / HBM_PEAK_GBS * 100, 2),
        "tokens_per_s": round(bsz * L / total, 1),
        # secondary: reference-formula flop rate of the fwd + VJP pair
        "ref_formula_TFLOPs": round(REF_FLOP_PER_ELEMENT * bsz * L * D * N / total / 1e12, 3),
    }
    # the same fwd + VJP pair replayed from a captured HIP graph: no host
    # work between the launches, so this is the GPU time of the pair (at
    # small shapes the eager calls above also hold the host's launch time)
    try:
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            y, ck = scan.scan_forward(*args, save_ckpt=True)
            scan.scan_backward(*args, g4, ckpt=ck)
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y, ck = scan.scan_forward(*args, save_ckpt=True)
            scan.scan_backward(*args, g4, ckpt=ck)
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            graph.replay()
        torch.cuda.synchronize()
        tg = (time.perf_counter() - t0) / iters
        out["graph_fwd_vjp_us"] = round(tg * 1e6, 2)
        out["graph_GBps"] = round((bf + bb) / tg / 1e9, 1)
        out["graph_pct_hbm_peak"] = round((bf + bb) / tg / 1e9 / HBM_PEAK_GBS * 100, 2)
        out["graph_tokens_per_s"] = round(bsz * L / tg, 1)
    except RuntimeError as err:
        print(f"bench.py: scan graph capture failed ({err})", file=sys.stderr, flush=True)
    return out


def step_scan_inputs(torch, device):
    """The fused scan call of one VisionMamba-2D layer of the step, in the
    block's layouts: B=32, K=4 directions of a 14x14 grid (L=196), D=768,
    N=16, dt_rank 24, fp32; u and delta_raw direction-major (K, B*L, D),
    B and C column slices of the x_proj output (K, B*L, 24 + 2N), z the
    second half of the in_proj output (B, L, K, 2D)."""
    from mlx_vision_mamba_amd import directions
    bsz, L, K, D, N, R = 32, 196, 4, 768, 16, 24
    g = torch.Generator().manual_seed(0)

    def bnkd(t):
        return t.view(K, bsz, L, t.shape[-1]).permute(1, 2, 0, 3)

    u = torch.randn(K, bsz * L, D, generator=g).to(device)
    draw = (torch.randn(K, bsz * L, D, generator=g) * 0.5 - 4.6).to(device)
    bias = (torch.randn(K, D, generator=g) * 0.1).to(device)
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(K, D, 1).to(device)
    dbc = torch.randn(K, bsz * L, R + 2 * N, generator=g).to(device)
    bc = bnkd(dbc)
    Dv = torch.ones(K, D, device=device)
    xz = torch.randn(bsz, L, K, 2 * D, generator=g).to(device)
    dy = torch.randn(bsz, L, K, D, generator=g).to(device)
    tok = directions.seq_to_tok_table(K, L, (14, 14)).to(device)
    args = (bnkd(u), bnkd(draw), bias, A, bc[..., R:R + N], bc[..., R + N:], Dv, xz[..., D:])
    return args, dy, tok


def scan_driver(torch, scan, device):
    """Profiling driver (--scan-driver): one 512 MiB device copy, whose HBM
    traffic is known and calibrates the byte counters, then two fused scan
    forward + VJP calls at the VisionMamba step shape."""
    src = torch.empty(128 * 1024 * 1024, dtype=torch.float32, device=device).uniform_()
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    args, dy, tok = step_scan_inputs(torch, device)
    dxz = torch.empty(args[7].shape[:3] + (2 * args[7].shape[3],), device=device)
    d_dbc = torch.empty(args[4].shape[2], args[4].shape[0] * args[4].shape[1],
                        args[4].stride(1), device=device)
    R, N = 24, args[3].shape[-1]
    dbc_v = d_dbc.view(d_dbc.shape[0], args[4].shape[0], args[4].shape[1], -1).permute(1, 2, 0, 3)
    for _ in range(2):
        y, y_raw, ck = scan.scan_fused_forward(*args, tok=tok, save=True)
        scan.scan_fused_backward(*args, y_raw, ck, dy, tok=tok, dB=dbc_v[..., R:R + N],
                                 dC=dbc_v[..., R + N:], dz=dxz[..., args[7].shape[3]:])
    torch.cuda.synchronize()
    print(json.dumps({"scan_driver": "done", "shape": "B=32 L=196 K=4 D=768 N=16 fp32 fused"}),
          flush=True)


def scan_driver_long(torch, scan, device):
    """Profiling driver (--scan-driver-long): the same 512 MiB calibration
    copy, then two plain scan forward + VJP calls at B=8, L=16384, D=1536,
    N=16 with bf16 u / B / C / y / gradients (the long-sequence case)."""
    from mlx_vision_mamba_amd import synthetic as scan_inputs
    src = torch.empty(128 * 1024 * 1024, dtype=torch.float32, device=device).uniform_()
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    u, dl, A, Bm, Cm, Dv, g = [t.to(device) for t in scan_inputs.make(8, 16384, 1536, 16, seed=0,
                                                                         dtype=torch.bfloat16)]
    args = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
            Dv.unsqueeze(0))
    for _ in range(2):
        y, ck = scan.scan_forward(*args, save_ckpt=True)
        scan.scan_backward(*args, g.unsqueeze(2), ckpt=ck)
    torch.cuda.synchronize()
    print(json.dumps({"scan_driver": "done", "shape": "B=8 L=16384 D=1536 N=16 bf16"}), flush=True)


def scan_driver_small(torch, scan, device):
    """Profiling driver (--scan-driver-small): the single-block scan at B=2,
    L=196, D=1536, N=16 fp32, forward + VJP captured in one HIP graph and
    replayed 20 times (the launch sequence of the graph figure of the bench
    line's single-block entry)."""
    from mlx_vision_mamba_amd import synthetic as scan_inputs
    u, dl, A, Bm, Cm, Dv, g = [t.to(device) for t in scan_inputs.make(2, 196, 1536, 16, seed=0)]
    args = (u.unsqueeze(2), dl.unsqueeze(2), A.unsqueeze(0), Bm.unsqueeze(2), Cm.unsqueeze(2),
            Dv.unsqueeze(0))
    g4 = g.unsqueeze(2)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        y, ck = scan.scan_forward(*args, save_ckpt=True)
        scan.scan_backward(*args, g4, ckpt=ck)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y, ck = scan.scan_forward(*args, save_ckpt=True)
        scan.scan_backward(*args, g4, ckpt=ck)
    for _ in range(20):
        graph.replay()
    torch.cuda.synchronize()
    print(json.dumps({"scan_driver": "done", "shape": "B=2 L=196 D=1536 N=16 fp32, 20 graph replays"}),
          flush=True)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "scan_visionmamba_shape_traffic_pmc.md")
LONG_PROFILE = os.path.join(ROOT, "profiles", "scan_long_bf16_pmc.md")
LONG_PASSES = ("fwd_aggregate", "fwd_main", "bwd_aggregate", "bwd_main")


def measured_traffic(key, kind=int, path=TRAFFIC_PROFILE):
    """A figure measured with rocprofv3 counters (a line `key: <value>` of a
    committed profile summary: HBM bytes per call from FETCH_SIZE /
    WRITE_SIZE, or a kernel's VALU busy fraction from the VALUBusy counter;
    by default the scan at the VisionMamba step shape), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return kind(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def cpu_baseline(torch):
    """Oracle VisionMamba step on the host cores: batch 2, one step."""
    from oracle import torch_ref
    import mlx_vision_mamba_amd as mvm
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch.manual_seed(1001)
    model = mvm.VisionMamba(img_size=224, patch_size=16, in_channels=1, embed_dim=384, depth=6,
                            d_state=16, input_dim=2)
    params = {k: v.detach().clone().requires_grad_(True) for k, v in model.named_parameters()}
    x = torch.randn(2, 224, 224, 1, generator=torch.Generator().manual_seed(1))

    def step():
        for p in params.values():
            p.grad = None
        out = torch_ref.vision_mamba(params, x, input_dim=2, patch_size=16, depth=6,
                                     grid_shape=(14, 14), d_state=16, d_conv=4)
        out.mean().backward()

    step()  # warm-up
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[2]
    scan_cpu = cpu_scan_baseline(torch)
    return {"value": round(2 / dt, 3), "unit": "imgs/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": "VisionMamba-2D K=4 step (fwd + mean loss + bwd), batch 2 of the same "
                      "224x224x1 / patch 16 / E=384 / depth 6 model, float32, reference's "
                      "sequential scan restated in torch; 1 warm-up, median of 5 timed steps",
            "seconds_per_step": round(dt, 2), "step_seconds": [round(t, 2) for t in times],
            "scan": scan_cpu}


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_scan_baseline(torch):
    """The reference's sequential and chunked scans (restated in torch,
    materialised discretisation, per-step loop) forward + VJP on the host at
    B=2, L=196, D=1536, N=16 fp32: 1 warm-up, median of 5; and the
    sequential scan on a slice of B=8, L=16384 (cpu_long_slice)."""
    from oracle import torch_ref
    from mlx_vision_mamba_amd import synthetic as scan_inputs
    from mlx_vision_mamba_amd.scan import algorithmic_bytes
    u, dl, A, Bm, Cm, Dv, g = scan_inputs.make(2, 196, 1536, 16, seed=0)
    nbytes = sum(algorithmic_bytes(2, 196, 1536, 16, 4, 4))
    out = {}
    for name, fn in (("sequential", torch_ref.scan_sequential), ("chunked", torch_ref.scan_chunked)):
        times = []
        for _ in range(6):
            ins = [t.clone().requires_grad_(True) for t in (u, dl, A, Bm, Cm, Dv)]
            t0 = time.perf_counter()
            y = fn(*ins)
            torch.autograd.grad(y, ins, g)
            times.append(time.perf_counter() - t0)
        med = sorted(times[1:])[2]
        out[name] = {"fwd_vjp_ms": round(med * 1e3, 2), "GBps": round(nbytes / med / 1e9, 3)}
    out["shape"] = "B=2 L=196 D=1536 N=16 fp32"
    out["long_B8_L16384_slice"] = cpu_long_slice(torch)
    return out


def cpu_long_slice(torch):
    """The reference's sequential scan (restated in torch) forward + VJP at
    B=8, L=16384, N=16 on an exact slice of 96 of the 1536 channels (the
    channels are independent), fp32 arithmetic on bf16-rounded u / B / C,
    timed once.  The full width would hold ~60 GB of materialised
    discretisation; the slice time x 16 is reported as an upper bound on the
    full-width time (the per-step Python and dispatch overhead does not grow
    with the width).  The chunked restatement's VJP takes ~3x longer here
    and is left out to bound the run."""
    from oracle import torch_ref
    from mlx_vision_mamba_amd import synthetic as scan_inputs
    from mlx_vision_mamba_amd.scan import algorithmic_bytes
    ins = [t.float() for t in scan_inputs.make(8, 16384, 96, 16, seed=4, dtype=torch.bfloat16)]
    u, dl, A, Bm, Cm, Dv, g = ins
    leaves = [t.clone().requires_grad_(True) for t in (u, dl, A, Bm, Cm, Dv)]
    t0 = time.perf_counter()
    y = torch_ref.scan_sequential(*leaves)
    torch.autograd.grad(y, leaves, g)
    dt = time.perf_counter() - t0
    full = sum(algorithmic_bytes(8, 16384, 1536, 16, 2, 2))
    return {"mode": "sequential", "slice": "B=8 L=16384 D=96 of 1536 N=16",
            "slice_fwd_vjp_s": round(dt, 2), "scaled_fwd_vjp_s": round(16 * dt, 1),
            "GBps_at_scaled_time": round(full / (16 * dt) / 1e9, 3),
            "note": "scaled x16 from the slice: an upper bound on the full-width time"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="time the eager step loop instead of replays of the captured HIP graph")
    ap.add_argument("--tune-gemms", metavar="CSV", default=None,
                    help="tune the step's GEMMs with TunableOp (2 steps) and write the picks to CSV")
    ap.add_argument("--default-gemms", action="store_true",
                    help="library-default GEMM selections (ignore the recorded MI355X picks)")
    ap.add_argument("--scan-driver", action="store_true",
                    help="profiling driver only: a 512 MiB copy + 2 scan fwd/VJP calls at the "
                         "VisionMamba step shape")
    ap.add_argument("--scan-driver-long", action="store_true",
                    help="profiling driver only: a 512 MiB copy + 2 plain scan fwd/VJP calls at "
                         "B=8 L=16384 D=1536 N=16 bf16")
    ap.add_argument("--scan-driver-small", action="store_true",
                    help="profiling driver only: 20 graph replays of the scan fwd/VJP pair at "
                         "B=2 L=196 D=1536 N=16 fp32")
    ap.add_argument("--no-encoders", action="store_true",
                    help="skip the 3D (K=6) and 4D (K=8) encoder steps")
    ap.add_argument("--torch-adamw", action="store_true",
                    help="update with torch's fused AdamW instead of the package's one-launch "
                         "AdamW")
    args = ap.parse_args()
    global TORCH_ADAMW
    TORCH_ADAMW = args.torch_adamw
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the selective-scan path is benchmarked on a "
              "single MI355X; run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import mlx_vision_mamba_amd as mvm
    from mlx_vision_mamba_amd import scan

    from mlx_vision_mamba_amd import gemm_tuning

    device = torch.device("cuda:0")
    if args.scan_driver:
        scan_driver(torch, scan, device)
        return
    if args.scan_driver_long:
        scan_driver_long(torch, scan, device)
        return
    if args.scan_driver_small:
        scan_driver_small(torch, scan, device)
        return
    if args.tune_gemms:
        gemm_tuning.start_tuning(args.tune_gemms)
        bench_step(torch, mvm, scan, 2, 1, device, graph=False)
        print(json.dumps({"tuned_gemms": args.tune_gemms}), flush=True)
        return
    tuned = False if args.default_gemms else gemm_tuning.load()
    value_region, eager, per, mode = bench_step(torch, mvm, scan, args.steps, args.warmup, device,
                                                graph=not args.eager)
    elapsed, enqueued = value_region["elapsed"], value_region["issued"]
    imgs = 32 * args.steps / elapsed

    bwd = per["bwd"]
    bwd_t = sum(t for t, _ in bwd) / len(bwd)
    bwd_b = sum(b for _, b in bwd) / len(bwd)
    fwd = per["fwd"]
    fwd_t = sum(t for t, _ in fwd) / len(fwd)
    fwd_b = sum(b for _, b in fwd) / len(fwd)
    achieved = bwd_b / bwd_t / 1e9
    roofline = {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": measured_traffic("bwd_call_hbm_bytes"),
        # traffic and valu_busy_per_simd are not measured by this run: they
        # are read from the committed rocprofv3 counter summary named here
        "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT) + " (rocprofv3 FETCH_SIZE / "
                          "WRITE_SIZE, committed summary; not measured by this run)",
        "kernel": BWD_KERNELS,
        "algorithmic_bytes_per_launch": int(bwd_b), "avg_launch_us": round(bwd_t * 1e6, 2),
        "launches": len(bwd),
        "fwd_call": {"achieved": round(fwd_b / fwd_t / 1e9, 1), "avg_launch_us": round(fwd_t * 1e6, 2),
                     "algorithmic_bytes_per_launch": int(fwd_b)},
        # the backward is VALU-issue bound: share of the kernel's time the
        # SIMDs' VALU is issuing (VALUBusy counter, committed profile)
        "valu_busy_per_simd": measured_traffic("bwd_valu_busy_per_simd", float),
        "valu_busy_source": os.path.relpath(TRAFFIC_PROFILE, ROOT) + " (rocprofv3 VALUBusy, "
                            "committed summary; not measured by this run)",
        # secondary: the reference formula's flop rate over the fused fwd +
        # VJP calls (B*K = 128 scans of L = 196, D = 768, N = 16)
        "secondary_flops": secondary_flops(32 * 4 * 196 * 768 * 16, fwd_t + bwd_t),
        # a plain device copy on the same GPU: the practical HBM ceiling
        "copy_GBps": copy_bandwidth(torch, device),
    }
    scans = {
        "single_block_B2_L196": bench_scan(torch, scan, 2, 196, 1536, 16, torch.float32, 200, device),
        "long_B8_L16384_bf16": bench_scan(torch, scan, 8, 16384, 1536, 16, torch.bfloat16, 5, device),
    }
    # each pass of the long scan is VALU-issue bound: the share of its cycles
    # the SIMDs' VALU is issuing (VALUBusy counter, committed profile)
    scans["long_B8_L16384_bf16"]["valu_busy_per_pass"] = {
        p: measured_traffic("long_valu_busy_" + p, float, LONG_PROFILE) for p in LONG_PASSES}
    scans["long_B8_L16384_bf16"]["valu_busy_source"] = (
        os.path.relpath(LONG_PROFILE, ROOT) + " (rocprofv3 VALUBusy, committed summary; not "
        "measured by this run)")
    out = {
        "metric": METRIC, "value": round(imgs, 2), "unit": "imgs/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        # host time to issue one step (python, autograd, launches): the step
        # is host-bound when this approaches ms_per_step
        "host_issue_ms_per_step": round(enqueued / args.steps * 1e3, 3),
        "execution": "HIP graph replay of the captured step" if mode == "graph" else mode,
        "eager_ms_per_step": round(eager["elapsed"] / args.steps * 1e3, 3),
        "eager_host_issue_ms_per_step": round(eager["issued"] / args.steps * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) images, random-init weights)",
        "config": {"workload": "VisionMamba-2D K=4 train step (fwd + mean loss + bwd + AdamW)",
                   "global_batch": 32, "image": "224x224x1", "patch": 16, "seq_len": 196,
                   "embed_dim": 384, "d_inner": 768, "d_state": 16, "depth": 6,
                   "directions": 4, "parallelism": "single GPU"},
        "gemm_selection": ("TunableOp picks " + os.path.relpath(gemm_tuning.DEFAULT_FILE, ROOT)
                           if tuned else "library default"),
        "optimizer": ("torch fused AdamW" if TORCH_ADAMW
                      else "one-launch AdamW (mlx_vision_mamba_amd.optim)"),
        "roofline": roofline,
        "scan": scans,
    }
    if not args.no_encoders:
        out["encoders"] = {name: bench_encoder(torch, mvm, scan, name, 5, 2, device)
                           for name in ENCODERS}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
