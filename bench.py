"""Benchmark of the MI355X MoE block (the BASELINE.json metric) on one GPU.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c2,c3,c4,c5] [--no-cpu]

A step is one MoE layer call (router -> top-k -> sort -> grouped gate_up -> grouped down
-> combine) on one batch of synthetic tokens with that layer's inputs already in HBM.
Layers cycle through L distinct weight sets (more bytes than L2 + MALL) so every step
streams its experts from HBM. The W warmup steps and the K timed steps are each captured
as one HIP graph of exactly that many layer calls (cycling the L layers); the timed region
is one replay of the K-call graph, bracketed by device synchronisations.

The headline workload is C2 (decode batch 1, H2048 E256 top-8 + shared, I=IS=512, bf16):
``value`` = microseconds per layer (lower is better). The same line carries the C3
(batch 64, Zipf(1.1) routing), C4 (4096-token prefill) and C5 (40-layer fp8 stack at
batch 32) results, the roofline of the dominant kernel (the gate_up launch the block uses
for that batch size, timed with HIP events on the stream it runs on) and the CPU baseline (the CPU torch oracle of
the reference path, timed on this host's cores on a bounded sample).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
H, E, K_TOP, I, IS = 2048, 256, 8, 512, 512
SEEDS = {"c2": 1000, "c3": 2000, "c4": 3000, "c5": 4000, "c4f8": 5000}
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"] if (ROOT / "BASELINE.json").exists() \
    else "MoE layer us + achieved HBM TB/s (% peak), E=256 top-8 h=2048, batch 1/64"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class NS:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def make_layer(torch, dev, seed, zipf=False, fp8=False):
    """One full-shape layer's weights on ``dev`` (bf16 ~ N(0, 0.02); fp8 per-row if asked)."""
    g = torch.Generator(device=dev).manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)

    router = rnd(E, H)
    v = None
    if zipf:
        r, v = load_pkg().synth.zipf_router(router.cpu(), seed=seed)
        v = v * load_pkg().synth.ZIPF_MU
        router = r.to(dev)
        v = v.to(dev)
    gu, dn = rnd(E, 2 * I, H), rnd(E, H, I)
    experts = NS(gate_up_proj=gu, down_proj=dn, num_experts=E)
    if fp8:
        pkg = load_pkg()
        q, s = pkg.fp8.quantize_rows(gu)
        experts.gate_up_proj, experts.gate_up_scale = q, s
        del gu
        q, s = pkg.fp8.quantize_rows(dn)
        experts.down_proj, experts.down_scale = q, s
        del dn
    mlp = NS(
        gate=NS(weight=router),
        shared_expert=NS(gate_proj=NS(weight=rnd(IS, H)), up_proj=NS(weight=rnd(IS, H)),
                         down_proj=NS(weight=rnd(H, IS))),
        shared_expert_gate=NS(weight=rnd(1, H)),
        experts=experts,
    )
    return mlp, v


_PKG = None


def load_pkg():
    global _PKG
    if _PKG is None:
        import __graft_entry__

        _PKG = __graft_entry__.load_package()
    return _PKG


def layer_bytes(D, T, fp8=False):
    """Algorithmic HBM bytes of one layer: each distinct expert's weights once (+ fp32 row
    scales for fp8), the shared expert, the router | shared-gate rows, the token rows in and
    the output rows out. Nothing an implementation chooses to write and read back."""
    per_expert = 3 * I * H * (1 if fp8 else 2) + (3 * I * 4 if fp8 else 0)
    weights = D * per_expert + 3 * IS * H * 2 + (E + 1) * H * 2
    return weights + T * H * 2 * 2


def impl_bytes(T, decode):
    """This implementation's own intermediate round trips per layer (written, then read
    back): the activations act [T*k, I] and act_sh [T, IS], the router logits, and in the
    tiled / prefill regimes the pair outputs y [T*k, H] and y_sh [T, H] that the combine
    reads."""
    b = (T * K_TOP * I + T * IS) * 2 * 2 + T * 320 * 2 * 2
    if not decode:
        b += (T * K_TOP * H + T * H) * 2 * 2
    return b


def gate_up_bytes(D, T, fp8=False, logits=False):
    """Algorithmic bytes of one gate_up launch: each distinct expert's gate/up rows once
    (+ fp32 row scales), the shared expert's gate/up rows, the token rows, the activations
    written; with ``logits`` also the router logits the decode launch routes from."""
    per_expert = 2 * I * H * (1 if fp8 else 2) + (2 * I * 4 if fp8 else 0)
    b = D * per_expert + 2 * IS * H * 2 + T * H * 2 + T * K_TOP * I * 2 + T * IS * 2
    if logits:
        b += T * 320 * 2  # logits rows [T, n_pack = 320]
    return b


def capture(torch, fn):
    """A HIP graph of ``fn()`` on a side stream (torch's capture)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm the caching allocator outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps, warmup, pre=None):
    """ms of ``reps`` replays of ``g`` after ``warmup`` untimed ones (and one of ``pre``)."""
    if pre is not None:
        pre.replay()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop)  # ms


_ACC_SAMPLE: dict = {}


def run_config(torch, dev, name, T, layers, steps, warmup, zipf=False, fp8=False):
    """Times ``steps`` layer calls of config ``name``; returns a result dict."""
    pkg = load_pkg()
    t0 = time.time()
    mlps, xs = [], []
    for li in range(layers):
        mlp, v = make_layer(torch, dev, seed=SEEDS[name] + li, zipf=zipf, fp8=fp8)
        g = torch.Generator(device=dev).manual_seed(li + 7)
        x = torch.randn(T, H, generator=g, device=dev)
        if v is not None:
            x = x + v[None, :]  # v already scaled by the Zipf construction's mu
        mlps.append(mlp)
        xs.append(x.to(torch.bfloat16))
        pkg.block.pack_router(mlp)
    torch.cuda.synchronize()
    log(f"[{name}] {layers} layers ready in {time.time() - t0:.1f}s")

    # routing statistics (outside the timed region)
    Ds, ok = [], True
    for mlp, x in zip(mlps, xs):
        out, idx, _, _ = pkg.block.moe(x, mlp, K_TOP, return_routing=True)
        Ds.append(int(torch.unique(idx).numel()))
        ok = ok and bool(torch.isfinite(out.float()).all())
    torch.cuda.synchronize()
    D = sum(Ds) / len(Ds)
    # the GPU result of layer 0 for the CPU leg's accuracy check (cpu_baseline)
    mlp, x = mlps[0], xs[0]
    out, idx, wts, logits = pkg.block.moe(x, mlp, K_TOP, decode=T <= 64, return_routing=True)
    sh, ex = mlp.shared_expert, mlp.experts
    w0 = {"router": mlp.gate.weight, "gate_up": ex.gate_up_proj, "down": ex.down_proj,
          "sh_gate": sh.gate_proj.weight, "sh_up": sh.up_proj.weight,
          "sh_down": sh.down_proj.weight, "sh_gate_w": mlp.shared_expert_gate.weight}
    if fp8:
        w0.update(gate_up_scale=ex.gate_up_scale, down_scale=ex.down_scale)
    _ACC_SAMPLE[name] = dict(x=x.cpu(), out=out.cpu(), idx=idx.cpu(), wts=wts.cpu(),
                             logits=logits.cpu(), w=w0, fp8=fp8, decode=T <= 64)
    del out, idx, wts, logits

    def calls(n):
        # n layer calls, cycling the L distinct layers
        def run():
            for i in range(n):
                pkg.block.moe(xs[i % layers], mlps[i % layers], K_TOP, decode=T <= 64)
        return run

    # exactly `steps` timed layer calls after `warmup` untimed ones, each a graph of its own
    graph = capture(torch, calls(steps))
    wgraph = capture(torch, calls(warmup)) if warmup > 0 else None
    ms = time_graph(torch, graph, 1, 0, pre=wgraph)
    nsteps = steps
    us_layer = ms * 1000.0 / nsteps
    reps = max(1, -(-steps // layers))
    wreps = max(1, -(-warmup // layers))
    lbytes = sum(layer_bytes(d, T, fp8) for d in Ds) / len(Ds)
    res = {
        "T": T, "layers": layers, "steps": nsteps, "warmup": warmup,
        "us_per_layer": round(us_layer, 3),
        "tokens_per_s": round(T / (us_layer * 1e-6), 1), "distinct_experts": round(D, 2),
        "layer_bytes": int(lbytes), "layer_TBps": round(lbytes / (us_layer * 1e-6) / 1e12, 3),
        "layer_hbm_frac": round(lbytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "impl_bytes": impl_bytes(T, pkg.ops.decode_fits(T, H, E, K_TOP, I, IS)),
        "finite": ok, "weights": "fp8_e4m3" if fp8 else "bf16",
    }
    if T >= 1024:
        flops = 2 * T * K_TOP * 3 * I * H + 2 * T * 3 * IS * H + 2 * T * (E + 1) * H
        res["tflops"] = round(flops / (us_layer * 1e-6) / 1e12, 2)
        res["mfma_frac_bf16"] = round(flops / (us_layer * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4)
    del graph, wgraph

    if T <= 4:
        # the decoder layer's post-attention add + RMSNorm in front of the block: fused into
        # the router launch against its own launch followed by the block (not the headline)
        hs = [x.flip(0).roll(1, 1) for x in xs]
        nw = (torch.randn(H, generator=torch.Generator().manual_seed(3)) * 0.1).to(
            torch.bfloat16).to(dev)

        def fused_pass():
            for mlp, x, h in zip(mlps, xs, hs):
                pkg.block.add_rms_moe(x, h, nw, 1e-6, mlp, K_TOP, decode=True)

        def separate_pass():
            for mlp, x, h in zip(mlps, xs, hs):
                total, norm = pkg.ops.add_rms(x, h, nw, 1e-6)
                pkg.block.moe(norm, mlp, K_TOP, decode=True, residual=total)

        for key, fn in (("add_rms_moe_us", fused_pass), ("add_rms_then_moe_us", separate_pass)):
            graph = capture(torch, fn)
            res[key] = round(time_graph(torch, graph, reps, wreps) * 1000.0 / (reps * layers), 3)
            del graph

    # the dominant kernel alone, as the block launches it: the decode gate_up (routing in the
    # launch, routed experts + the shared expert's gate/up rows) for decode-path shapes, else
    # the grouped gate_up (routed + shared) over the sorted tile table
    decode = pkg.ops.decode_fits(T, H, E, K_TOP, I, IS)
    sps = []
    for mlp, x in zip(mlps, xs):
        logits = pkg.ops.router_logits(x, pkg.block.pack_router(mlp))
        if decode:
            sps.append(logits)
        else:
            _, idx, _ = pkg.ops.route(logits, K_TOP, experts=E)
            sps.append(pkg.ops.sort_pairs(idx, E, shared=True))
    torch.cuda.synchronize()

    def gate_up_pass():
        for mlp, x, sp in zip(mlps, xs, sps):
            ex = mlp.experts
            scale = getattr(ex, "gate_up_scale", None)
            if decode:
                pkg.ops.decode_gate_up(x, ex.gate_up_proj, K_TOP, logits=sp, experts=E,
                                       scale=scale,
                                       shared=(mlp.shared_expert.gate_proj.weight,
                                               mlp.shared_expert.up_proj.weight))
            else:
                pkg.ops.grouped_gate_up(x, K_TOP, ex.gate_up_proj, sp, scale=scale,
                                        shared=(mlp.shared_expert.gate_proj.weight,
                                                mlp.shared_expert.up_proj.weight))

    graph = capture(torch, gate_up_pass)
    ms = time_graph(torch, graph, reps, wreps)
    us_k = ms * 1000.0 / (reps * layers)
    kbytes = sum(gate_up_bytes(d, T, fp8, logits=decode) for d in Ds) / len(Ds)
    res["gate_up_kernel"] = "k_dec_gate_up" if decode else (
        ("k_prefill_gemm_f8" if fp8 else "k_prefill_gemm") if T > 512 else "k_expert_gemm")
    res["gate_up_us"] = round(us_k, 3)
    res["gate_up_bytes"] = int(kbytes)
    res["gate_up_GBps"] = round(kbytes / (us_k * 1e-6) / 1e9, 1)
    del graph, sps, mlps, xs
    torch.cuda.empty_cache()
    log(f"[{name}] {json.dumps(res)}")
    return res


def small_batches(torch, dev, layers=8, reps=20):
    """µs per layer of decode steps of 2-16 tokens (bf16 and fp8 experts, ``layers`` layers
    cycled, graph-replayed): the range between the C2 and C3 / C5 workloads, where the
    block picks between the decode kernels and the tiled expert GEMM."""
    pkg = load_pkg()
    out = {}
    for fp8 in (False, True):
        mlps = [make_layer(torch, dev, seed=700 + li, fp8=fp8)[0] for li in range(layers)]
        for mlp in mlps:
            pkg.block.pack_router(mlp)
        for T in (2, 4, 8, 16):
            g = torch.Generator(device=dev).manual_seed(T)
            xs = [torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16) for _ in mlps]

            def step():
                for mlp, x in zip(mlps, xs):
                    pkg.block.moe(x, mlp, K_TOP, decode=True)

            graph = capture(torch, step)
            us = time_graph(torch, graph, reps, 4) * 1000.0 / (reps * layers)
            out[f"{'fp8' if fp8 else 'bf16'}_T{T}"] = round(us, 2)
            del graph
        del mlps
        torch.cuda.empty_cache()
    log(f"[batches] {json.dumps(out)}")
    return out


def hbm_ceiling(torch, dev, gib=4, reps=10):
    """What library streaming kernels reach on this HBM, as a practical ceiling beside the
    8 TB/s peak: torch's sum over a gib-GiB bf16 tensor (reads only) and torch's copy of
    gib/2 GiB into another tensor (reads and writes gib GiB in all). Best of 5 timings of
    reps calls each, eager (the calls are milliseconds long)."""
    n = (gib << 30) // 2
    x = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_()
    out = {}

    def best(fn, nbytes):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t = []
        for _ in range(5):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                fn()
            b.record()
            torch.cuda.synchronize()
            t.append(a.elapsed_time(b) / reps)
        return round(nbytes / (min(t) * 1e-3) / 1e12, 3)

    out["read_sum_TBps"] = best(lambda: x.sum(), n * 2)
    # the probe library's plain streaming read (probe/stream_read.hip), over grid sizes
    import ctypes

    lib = ctypes.CDLL(str(ROOT / "qwen36-mi250-tracelab-20261107_amd" / "libmoe_probe.so"))
    fn = lib.moe_probe_stream_read
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sink = torch.empty(16384 * 256, dtype=torch.int32, device=dev)
    probe = {}
    for blocks in (1024, 2048, 4096, 8192, 16384):
        def read(b=blocks):
            if fn(x.data_ptr(), n * 2, sink.data_ptr(), b, stream) != 0:
                raise RuntimeError("moe_probe_stream_read failed")
        probe[str(blocks)] = best(read, n * 2)
    out["read_probe_TBps"] = max(probe.values())
    out["read_probe_by_workgroups"] = probe
    half = x[: n // 2]
    dst = torch.empty_like(half)
    out["copy_TBps"] = best(lambda: dst.copy_(half), n * 2)
    out["GiB_per_call"] = gib
    del x, dst
    torch.cuda.synchronize()
    return out


def cpu_baseline(torch, seconds):
    """The CPU torch restatement of the reference path (oracle.block_bf16: Transformers
    block with batched_mm experts, engine/experts.py) on C2, timed on this host."""
    from oracle import moe_oracle as orc

    w = orc.make_weights(H, E, I, IS, seed=0)
    g = torch.Generator().manual_seed(1)
    xs = [torch.randn(1, H, generator=g).to(torch.bfloat16) for _ in range(8)]
    orc.block_bf16(xs[0], w, K_TOP)  # warm
    n, t0 = 0, time.perf_counter()
    times = []
    while time.perf_counter() - t0 < seconds:
        t1 = time.perf_counter()
        orc.block_bf16(xs[n % len(xs)], w, K_TOP)
        times.append(time.perf_counter() - t1)
        n += 1
    times.sort()
    med = times[len(times) // 2]
    others = {}
    for name, T in (("c3", 64), ("c4", 4096)):
        # the same CPU path at the other batch sizes, a few calls each (bounded sample;
        # C3 with plain random routing, C5 is C3-like at 32 tokens with bf16 weights)
        xb = torch.randn(T, H, generator=g).to(torch.bfloat16)
        orc.block_bf16(xb, w, K_TOP)
        ts, tb = [], time.perf_counter()
        while len(ts) < 3 or (time.perf_counter() - tb < seconds / 3 and len(ts) < 50):
            t1 = time.perf_counter()
            orc.block_bf16(xb, w, K_TOP)
            ts.append(time.perf_counter() - t1)
        ts.sort()
        others[name] = {"T": T, "us_per_layer": round(ts[len(ts) // 2] * 1e6, 1), "calls": len(ts)}
    acc = {}
    for name, sm in _ACC_SAMPLE.items():
        # the same check the parity tests make, on each config's own layer 0: the GPU output
        # and (bf16 experts) the reference torch path on the same routing against the fp32
        # oracle; fp8 experts against the oracle on the dequantised weights
        lg = sm["logits"][:, :E].float()
        f32 = orc.block_fp32(sm["x"], sm["w"], sm["idx"], logits=lg)

        def mrel(a, b):
            return float((a.float() - b).abs().mean() / b.abs().mean())

        a = {"tokens": int(sm["x"].shape[0]),
             "max_abs_vs_fp32": round(float((sm["out"].float() - f32).abs().max()), 6),
             "mean_rel_vs_fp32": round(mrel(sm["out"], f32), 6)}
        if sm["fp8"]:
            a["bar"] = "fp8 experts against the fp32 oracle on the dequantised weights: " \
                       "max-abs 2e-2, mean-rel 6e-3"
        else:
            wc, ic = orc.compact_experts(sm["w"], sm["idx"])
            ref = orc.block_bf16_routed(sm["x"], wc, ic, sm["wts"], sm["logits"][:, E:E + 1],
                                        decode=sm["decode"])
            a["mean_rel_ref_path_vs_fp32"] = round(mrel(ref, f32), 6)
            a["bar"] = "max-abs 2e-2; mean-rel 5e-3, or 1.1x the reference path's own " \
                       "mean-rel where that exceeds 5e-3 (its bf16 rounding points alone do)"
        acc[name] = a
    return {
        "accuracy": acc or None,
        "value": round(med * 1e6, 1), "unit": "us/layer", "cores": torch.get_num_threads(),
        "affinity_cores": len(os.sched_getaffinity(0)), "kind": "port",
        "sample": f"C2 decode batch 1, {n} layer calls of the bf16 CPU torch path "
                  f"(oracle.block_bf16 = Transformers block + batched_mm experts) over "
                  f"{seconds:.0f}s, median",
        "other_batches": others,
    }


def head_name(results):
    return "c2" if "c2" in results else next(iter(results))


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.json"


def measured_traffic(kernel, config):
    """HBM bytes per launch of ``kernel`` on ``config`` from the committed counter summary
    (two rocprofv3 --pmc runs, summarised by --pmc-summary), or None."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    # the largest launch of that kernel family on that workload (the gate_up of the block)
    recs = [v for k, v in data.items()
            if k.startswith(f"{config}:moe::{kernel}<") and isinstance(v, dict)]
    if not recs:
        return None
    rec = max(recs, key=lambda v: v["hbm_bytes_per_launch"])
    return {"bytes_per_launch": rec["hbm_bytes_per_launch"],
            "source": f"profiles/{TRAFFIC_FILE.name} ({rec['command']})"}


def _pmc_rows(d, counter):
    import csv
    import glob

    out = {}
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            name = r["Kernel_Name"]
            out.setdefault(name, []).append(float(r["Counter_Value"]))
    return out


def pmc_summary(fetch_dir, write_dir, copy_mib, config):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch, as rocprofv3 reports them) of each moe::
    kernel, scaled by the counter's reading for the plain copy of ``copy_mib`` MiB, which
    reads and writes exactly that many bytes. Writes profiles/hbm_traffic.json and a
    markdown table."""
    fetch = _pmc_rows(fetch_dir, "FETCH_SIZE")
    write = _pmc_rows(write_dir, "WRITE_SIZE")
    n = copy_mib << 20

    def copy_of(rows):
        # the device-to-device copy of the calibration (torch copy_ -> HIP's copy kernel)
        cands = [(k, v) for k, v in rows.items() if "copybuffer" in k.lower()]
        k, v = max(cands, key=lambda kv: max(kv[1]))
        return k, max(v) * 1024.0

    ck, cf = copy_of(fetch)
    _, cw = copy_of(write)
    f_fac, w_fac = n / cf, n / cw
    cmd_base = (f"rocprofv3 --pmc {{}} --output-format csv -- python3 bench.py --calibrate-copy "
                f"{copy_mib} --configs {config} --no-cpu --steps 16 --warmup 16")
    data = {"copy_kernel": ck, "copy_bytes": n, "fetch_factor": f_fac, "write_factor": w_fac}
    lines = [f"# HBM traffic per launch ({config}), from FETCH_SIZE and WRITE_SIZE\n",
             "Commands (from the repository root on one MI355X; one counter per run):\n",
             "    " + cmd_base.format("FETCH_SIZE"), "    " + cmd_base.format("WRITE_SIZE"),
             f"    python3 bench.py --pmc-summary <fetch_dir> <write_dir> --pmc-copy-mib {copy_mib} "
             f"--pmc-config {config}\n",
             f"Calibration: the plain copy of {copy_mib} MiB (`{ck[:60]}`) reads {cf / 2**20:.1f} "
             f"MiB by FETCH_SIZE and writes {cw / 2**20:.1f} MiB by WRITE_SIZE: the counters are "
             f"scaled by {f_fac:.3f} (fetch) and {w_fac:.3f} (write).\n",
             "| kernel | launches | fetch MB | write MB | HBM MB per launch |", "|---|---|---|---|---|"]
    for k in sorted(fetch):
        if "moe::" not in k:
            continue
        fv = sum(fetch[k]) / len(fetch[k]) * 1024.0 * f_fac
        wv = sum(write.get(k, [0.0])) / max(1, len(write.get(k, []))) * 1024.0 * w_fac
        short = k.replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
        data[f"{config}:{short}"] = {"kernel": short, "fetch_bytes": fv, "write_bytes": wv,
                                      "hbm_bytes_per_launch": int(fv + wv),
                                      "command": cmd_base.format("FETCH_SIZE|WRITE_SIZE")}
        lines.append(f"| `{short}` | {len(fetch[k])} | {fv / 1e6:.2f} | {wv / 1e6:.2f} | "
                     f"{(fv + wv) / 1e6:.2f} |")
    prev = {}
    try:
        prev = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        pass
    # this config's kernels are replaced, not merged (kernels since removed drop out)
    prev = {k: v for k, v in prev.items() if not k.startswith(f"{config}:")}
    prev.update(data)
    TRAFFIC_FILE.parent.mkdir(exist_ok=True)
    TRAFFIC_FILE.write_text(json.dumps(prev, indent=1, sort_keys=True) + "\n")
    md = ROOT / "profiles" / f"hbm_traffic_{config}.md"
    md.write_text("\n".join(lines) + "\n")
    print(md.read_text())


KERNEL_STATS_FILES = {"c2": ("moe_layer_c2_decode_b1_kernels",
                              "C2: MoE layer, decode batch 1 (H2048 E256 top-8 + shared, bf16), 16 "
                              "layers cycled"),
                       "c3": ("moe_layer_c3_decode_b64_zipf_kernels",
                              "C3: MoE layer, batch 64 with Zipf(1.1) routing (bf16), 16 layers "
                              "cycled"),
                       "c4": ("moe_layer_c4_prefill_4096_kernels",
                              "C4: MoE layer, 4096-token prefill chunk (bf16), 4 layers cycled"),
                       "c5": ("moe_layer_c5_fp8_b32_kernels",
                              "C5: 40-layer stack, fp8-e4m3 routed experts, batch 32"),
                       "c4f8": ("moe_layer_c4f8_prefill_4096_fp8_kernels",
                                "C4's 4096-token prefill chunk with fp8-e4m3 routed experts "
                                "(not a BASELINE config), 4 layers cycled")}


def kernel_stats_summary(prof_dir, config):
    """The library's kernels in a `rocprofv3 --kernel-trace --stats` run of `bench.py
    --configs <config> --no-cpu` (stdout of the run in <prof_dir>.json): calls and average /
    min / max duration, ordered by total time. Written to profiles/moe_layer_<config>_*.md."""
    import csv
    import glob
    import re

    name, title = KERNEL_STATS_FILES[config]
    f = glob.glob(os.path.join(prof_dir, "**", "*kernel_stats.csv"), recursive=True)[0]
    rows = []
    for r in csv.DictReader(open(f)):
        n = r["Name"].replace("(anonymous namespace)::", "")
        m = re.match(r"(?:void )?(moe::[A-Za-z0-9_]+(?:<[^>]*>)?)", n)
        if m:
            rows.append((m.group(1), int(r["Calls"]), float(r["AverageNs"]) / 1e3,
                         float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3,
                         float(r["TotalDurationNs"])))
    rows.sort(key=lambda x: -x[5])
    lines = [f"# {title}\n",
             "Command (run on one MI355X from the repository root; `cd /tmp && export "
             "TMPDIR=/tmp` first, paths absolute):\n",
             f"    rocprofv3 --kernel-trace --stats --output-format csv -d <out> -o run -- python3 "
             f"bench.py --configs {config} --no-cpu > <out>.json",
             f"    python3 bench.py --stats-summary <out> --stats-config {config}\n",
             "Kernel statistics (rocprofv3 kernel_stats.csv; libmoe_mi355x.so kernels only; "
             "microseconds). The run includes the untimed routing-statistics pass, graph warm-up "
             "and the dominant-kernel (gate_up) graph (and, at C2, the graphs of the add + RMSNorm "
             "side measurement), so call counts exceed the timed steps.\n",
             "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    lines += [f"| `{k}` | {n} | {a:.2f} | {mi:.2f} | {ma:.2f} |" for k, n, a, mi, ma, _ in rows]
    try:
        line = json.loads(Path(prof_dir + ".json").read_text().strip().splitlines()[-1])
        c = line["configs"][config]
        lines += ["", f"Same run, bench line for {config} (timed under the profiler): "
                      f"{c['us_per_layer']} us/layer, gate_up kernel `{c['gate_up_kernel']}` "
                      f"{c['gate_up_us']} us per launch, {c['gate_up_GBps']} GB/s algorithmic."]
    except (OSError, ValueError, KeyError):
        pass
    md = ROOT / "profiles" / f"{name}.md"
    md.write_text("\n".join(lines) + "\n")
    print(md.read_text())


def counter_summary(dirs, config, name, commands):
    """Per-kernel medians of the SQ counters in one or more `rocprofv3 --pmc` runs (one
    counter set per run) of `bench.py --configs <config>`, for the launches of each kernel
    with its largest grid (the block's routed launches; the shared expert's side launches
    of the same kernel have smaller grids), with the ratios read from them. Written to
    profiles/<name>.md."""
    import csv
    import glob
    import statistics

    vals = {}   # kernel -> counter -> [values]
    grids = {}  # kernel -> max grid
    rows = []
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if "moe::" not in r["Kernel_Name"]:
                    continue
                k = (r["Kernel_Name"].replace("void ", "").replace("(anonymous namespace)::", "")
                     .split("(")[0])
                g = int(r["Grid_Size"])
                rows.append((k, g, r["Counter_Name"], float(r["Counter_Value"])))
                grids[k] = max(grids.get(k, 0), g)
    for k, g, c, v in rows:
        if g == grids[k]:
            vals.setdefault(k, {}).setdefault(c, []).append(v)
    counters = sorted({c for kv in vals.values() for c in kv})
    kernels = sorted(vals, key=lambda k: -max(statistics.median(v) for v in vals[k].values()))
    med = {k: {c: statistics.median(vals[k][c]) for c in vals[k]} for k in kernels}
    lines = [f"# Counters of the {config} kernels\n",
             "Commands (from the repository root on one MI355X; `cd /tmp && export TMPDIR=/tmp` "
             "first, paths absolute; one counter set per run):\n"]
    lines += ["    " + c for c in commands]
    lines += [f"    python3 bench.py --counter-summary <dir> [<dir> ...] --counter-config {config} "
              f"--counter-name {name}\n",
              "Medians per dispatch over the launches of each kernel with its largest grid, as "
              "rocprofv3 reports them.\n",
              "| counter | " + " | ".join(f"`{k}`" for k in kernels) + " |",
              "|---|" + "---|" * len(kernels)]
    for c in counters:
        lines.append(f"| `{c}` | " + " | ".join(
            f"{med[k][c]:.4g}" if c in med[k] else "" for k in kernels) + " |")

    def ratio(k, a, b):
        m = med[k]
        return f"{m[a] / m[b]:.3f}" if a in m and b in m and m[b] else ""

    derived = [("SQ_WAIT_ANY / SQ_WAVE_CYCLES (share of wave time in s_waitcnt)", "SQ_WAIT_ANY",
                "SQ_WAVE_CYCLES"),
               ("SQ_INSTS_VALU / SQ_INSTS_VMEM_RD (VALU instructions per load instruction)",
                "SQ_INSTS_VALU", "SQ_INSTS_VMEM_RD"),
               ("SQ_INST_LEVEL_VMEM / SQ_WAVE_CYCLES (load instructions in flight per wave)",
                "SQ_INST_LEVEL_VMEM", "SQ_WAVE_CYCLES"),
               ("SQ_VALU_MFMA_BUSY_CYCLES / SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES",
                "SQ_BUSY_CYCLES"),
               ("TCP_TCC_READ_REQ_LATENCY_sum / TCP_TCC_READ_REQ_sum (cycles from a vector L1 "
                "miss to its L2 reply)", "TCP_TCC_READ_REQ_LATENCY_sum", "TCP_TCC_READ_REQ_sum"),
               ("TCC_EA0_RDREQ_LEVEL_sum / TCC_EA0_RDREQ_sum (cycles from an L2 miss to its "
                "memory reply)", "TCC_EA0_RDREQ_LEVEL_sum", "TCC_EA0_RDREQ_sum"),
               ("TCC_HIT_sum / TCC_REQ_sum (L2 hit rate)", "TCC_HIT_sum", "TCC_REQ_sum"),
               ("TCP_UTCL1_TRANSLATION_MISS_sum / TCP_UTCL1_REQUEST_sum (L1 TLB miss rate)",
                "TCP_UTCL1_TRANSLATION_MISS_sum", "TCP_UTCL1_REQUEST_sum")]
    lines += ["", "| ratio | " + " | ".join(f"`{k}`" for k in kernels) + " |",
              "|---|" + "---|" * len(kernels)]
    for label, a, b in derived:
        cells = [ratio(k, a, b) for k in kernels]
        if any(cells):
            lines.append(f"| {label} | " + " | ".join(cells) + " |")
    md = ROOT / "profiles" / f"{name}.md"
    md.write_text("\n".join(lines) + "\n")
    print(md.read_text())


def trace_summary(trace_dir, config):
    """Per-layer timeline of the timed graph replay from a `rocprofv3 --kernel-trace` run of
    `bench.py --configs <config> --no-cpu`: the library's dispatches sorted by start, split
    where the device idles more than 50 us, the longest such run kept (the timed replay);
    its period is where the first kernel name recurs. Per position of the period: median
    start offset from the layer's first kernel, duration, and the gap since the previous
    dispatch ended. Written to profiles/timeline_<config>.md."""
    import csv
    import statistics

    paths = sorted(Path(trace_dir).rglob("*kernel_trace.csv"))
    if not paths:
        raise SystemExit(f"no kernel_trace.csv under {trace_dir}")
    rows = []
    for path in paths:
        with open(path) as f:
            for r in csv.DictReader(f):
                if "moe::" in r["Kernel_Name"]:
                    name = (r["Kernel_Name"].replace("void ", "")
                            .replace("(anonymous namespace)::", "").split("(")[0])
                    rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), name,
                                 r.get("Queue_Id", "")))
    rows.sort()
    runs, cur = [], [rows[0]]
    for r in rows[1:]:
        if r[0] - max(c[1] for c in cur[-4:]) > 200_000:
            runs.append(cur)
            cur = []
        cur.append(r)
    runs.append(cur)
    run = max(runs, key=len)
    # layers: from one router launch to the next (with the shared expert on the auxiliary
    # stream the dispatch order inside a layer varies, so kernels are matched by name and
    # occurrence, not by position)
    # the routed chain's queue is the router's; a dispatch on another queue (the shared
    # expert on the auxiliary stream, forked at the block's start just before the router, and
    # the joining combine) belongs to the last layer whose router started at most 10 us after it
    mainq = next((r[3] for r in run if "router" in r[2]), "")
    rstarts = [r[0] for r in run if "router" in r[2]]
    segs = [[] for _ in rstarts]
    for r in run:
        lead = 0 if r[3] == mainq else 10_000
        i = max((j for j, t in enumerate(rstarts) if t <= r[0] + lead), default=-1)
        if 0 <= i < len(segs):
            segs[i].append(r)
    segs = [sorted(sg) for sg in segs[:-1]]

    def keyed(seg):
        seen, out = {}, []
        for r in seg:
            seen[r[2]] = seen.get(r[2], 0) + 1
            out.append((f"{r[2]}#{seen[r[2]]}", r[:3]))
        return out

    segs = [keyed(sg) for sg in segs]
    ref = sorted(k for k, _ in segs[len(segs) // 2]) if segs else []
    layers = [dict(sg) for sg in segs if sorted(k for k, _ in sg) == ref]
    layers = layers[1:-1] if len(layers) > 4 else layers  # drop the replay's ramp and tail
    starts = [min(r[0] for r in ly.values()) for ly in layers]
    per = statistics.median(b - a for a, b in zip(starts, starts[1:])) / 1e3 if len(starts) > 1 else 0
    first = next(k for k, _ in segs[len(segs) // 2])
    order = sorted(ref, key=lambda k: statistics.median(ly[k][0] - ly[first][0] for ly in layers))
    period = len(order)
    run = [r for ly in layers for r in ly.values()]
    lines = [f"# Timeline of one {config} layer in the timed graph replay\n",
             "Commands (from the repository root on one MI355X; `cd /tmp && export TMPDIR=/tmp` "
             "first, paths absolute):\n",
             f"    rocprofv3 --kernel-trace --output-format csv -d <out> -o run -- python3 bench.py "
             f"--configs {config} --no-cpu",
             f"    python3 bench.py --trace-summary <out> --trace-config {config}\n",
             f"{len(layers)} layers of the longest back-to-back run of library dispatches "
             f"({len(run)} dispatches); medians in microseconds. Layer period (first kernel "
             f"start to the next layer's first kernel start): **{per:.2f} us**.\n",
             "| # | kernel | start offset | duration | gap before (since previous dispatch ended) |",
             "|---|---|---|---|---|"]
    busy = 0.0
    for i, k in enumerate(order):
        off = statistics.median((ly[k][0] - min(r[0] for r in ly.values())) / 1e3 for ly in layers)
        dur = statistics.median((ly[k][1] - ly[k][0]) / 1e3 for ly in layers)
        gaps = []
        for j, ly in enumerate(layers):
            prev = [r[1] for r in ly.values() if r[0] < ly[k][0]]
            if not prev and j:
                prev = [r[1] for r in layers[j - 1].values()]
            if prev:
                gaps.append((ly[k][0] - max(prev)) / 1e3)
        gap = statistics.median(gaps) if gaps else 0.0
        busy += dur
        lines.append(f"| {i} | `{k.split('#')[0]}` | {off:.2f} | {dur:.2f} | {gap:.2f} |")

    def covered(ly):  # time with at least one library kernel running
        iv = sorted((r[0], r[1]) for r in ly.values())
        tot, cs, ce = 0, iv[0][0], iv[0][1]
        for a, b in iv[1:]:
            if a > ce:
                tot += ce - cs
                cs, ce = a, b
            else:
                ce = max(ce, b)
        return (tot + ce - cs) / 1e3

    cov = statistics.median(covered(ly) for ly in layers) if layers else 0.0
    lines.append(f"\nSum of the medians of the kernel durations: {busy:.2f} us; time with at "
                 f"least one kernel running: {cov:.2f} us of the {per:.2f} us period (the rest, "
                 f"{per - cov:.2f} us, is time between dispatches). A negative gap is an overlap "
                 "(the dispatch started before the latest-ending earlier one ended: kernels on "
                 "the auxiliary stream).")
    md = ROOT / "profiles" / f"timeline_{config}.md"
    md.write_text("\n".join(lines) + "\n")
    print(md.read_text())


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--configs", default="c2,c3,c4,c5,c4f8,batches")
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first run a plain device copy of MIB MiB (the known-size kernel the "
                         "FETCH_SIZE / WRITE_SIZE counters are scaled by)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of "
                         "`bench.py --calibrate-copy M --configs c` into profiles/ and exit")
    ap.add_argument("--pmc-copy-mib", type=int, default=256)
    ap.add_argument("--pmc-config", default="c2")
    ap.add_argument("--trace-summary", metavar="TRACE_DIR",
                    help="summarise a rocprofv3 --kernel-trace run of `bench.py --configs c` "
                         "into profiles/timeline_<c>.md and exit")
    ap.add_argument("--trace-config", default="c2")
    ap.add_argument("--stats-summary", metavar="PROF_DIR",
                    help="summarise a rocprofv3 --kernel-trace --stats run of `bench.py "
                         "--configs c` into profiles/moe_layer_<c>_*.md and exit")
    ap.add_argument("--stats-config", default="c2")
    ap.add_argument("--counter-summary", nargs="+", metavar="PMC_DIR",
                    help="summarise rocprofv3 --pmc runs of `bench.py --configs c` into "
                         "profiles/<--counter-name>.md and exit")
    ap.add_argument("--counter-config", default="c4")
    ap.add_argument("--counter-name", default="counters")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="print the read (torch sum) and copy rates of library streaming "
                         "kernels on this GPU as one JSON line and exit")
    ap.add_argument("--counter-commands", nargs="*", default=[],
                    help="the rocprofv3 commands of the runs (quoted, for the summary)")
    args = ap.parse_args()
    if args.stats_summary:
        kernel_stats_summary(args.stats_summary, args.stats_config)
        return
    if args.counter_summary:
        counter_summary(args.counter_summary, args.counter_config, args.counter_name,
                        args.counter_commands)
        return
    if args.trace_summary:
        trace_summary(args.trace_summary, args.trace_config)
        return
    if args.pmc_summary:
        pmc_summary(args.pmc_summary[0], args.pmc_summary[1], args.pmc_copy_mib, args.pmc_config)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the MoE block runs "
              "on one GPU with no TP/EP exchange); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.hbm_ceiling:
        print(json.dumps({"hbm_ceiling": hbm_ceiling(torch, dev), "peak_TBps": HBM_PEAK_GBS / 1e3}))
        return
    pkg = load_pkg()
    pkg._lib.load()
    cfgs = [c.strip() for c in args.configs.split(",") if c.strip()]
    if args.calibrate_copy:
        n = args.calibrate_copy << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    results = {}
    if "c2" in cfgs:
        results["c2"] = run_config(torch, dev, "c2", 1, args.layers, args.steps, args.warmup)
    if "c3" in cfgs:
        results["c3"] = run_config(torch, dev, "c3", 64, args.layers, args.steps, args.warmup,
                                   zipf=True)
    if "c4" in cfgs:
        results["c4"] = run_config(torch, dev, "c4", 4096, 4, max(8, args.steps // 32),
                                   max(4, args.warmup // 8))
    if "c5" in cfgs:
        results["c5"] = run_config(torch, dev, "c5", 32, 40, max(40, args.steps // 40 * 40),
                                   40, fp8=True)
    if "c4f8" in cfgs:
        # not a BASELINE config: C4's prefill chunk with C5's fp8-e4m3 experts
        results["c4f8"] = run_config(torch, dev, "c4f8", 4096, 4, max(8, args.steps // 32),
                                     max(4, args.warmup // 8), fp8=True)
    if "batches" in cfgs:
        results["batches"] = small_batches(torch, dev)
    workloads = {k: v for k, v in results.items() if k != "batches"}
    if not workloads:
        raise SystemExit("bench.py: --configs needs at least one of c2, c3, c4, c5")
    head = workloads.get("c2") or next(iter(workloads.values()))
    cpu = None if args.no_cpu else cpu_baseline(torch, args.cpu_seconds)
    accuracy = cpu.pop("accuracy", None) if cpu else None
    kbytes, kus = head["gate_up_bytes"], head["gate_up_us"]
    achieved = kbytes / (kus * 1e-6) / 1e9
    traffic = measured_traffic(head["gate_up_kernel"], head_name(workloads))
    line = {
        "metric": METRIC,
        "value": head["us_per_layer"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": head["warmup"],
        "ms_per_step": round(head["us_per_layer"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (weights ~N(0,0.02) random-init, activations ~N(0,1))",
        "config": {"workload": "C2 MoE layer decode batch 1: H2048 E256 top-8 + shared, "
                               "I=IS=512, bf16, 16 distinct layers cycled",
                   "tokens": head["T"], "parallelism": "single GPU"},
        "hbm_TBps": head["layer_TBps"],
        "hbm_frac": head["layer_hbm_frac"],
        "tokens_per_s": head["tokens_per_s"],
        "roofline": {"bound": "hbm", "kernel": head["gate_up_kernel"],
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes_per_launch"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "bytes_per_launch": kbytes, "us_per_launch": kus},
        "cpu_baseline": cpu,
        "accuracy": accuracy,
        "configs": results,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
