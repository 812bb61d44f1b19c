#!/usr/bin/env python3
"""Benchmark of the MoE feed-forward layer on one MI355X.

    python bench.py [--steps K] [--warmup W] [--T 128] [--prefill-T 8192] [--no-cpu-baseline]
                    [--no-prefill] [--no-extra] [--copy-probe-mib N] [--only-extra TEXT]

Headline workload: the Qwen3-30B-A3B MoE layer (H=2048, E=128, top-8, I=768, bf16 weights
~N(0,0.02), activations ~N(0,1), synthetic, seed 0) at decode T=128. One step is one call of
the whole layer (router -> permute -> gate_up+SiLU*mul -> down -> combine) on inputs already
resident in HBM. The same run also measures the prefill chunk T=8192 with a Zipf(1.2)
router bias (skewed expert loads), and (under "extra") the decode sweep T=1..256, the
Qwen3-Next-style E=512 layer with a shared expert and its fp8-e4m3 variant.

Printed: one JSON line. `value` is the layer's algorithmic HBM throughput in GB/s at T=128
(hit experts' weights + router weight + x in + y out, divided by the wall time of back-to-back
calls). `roofline` describes the dominant kernel (gate_up), timed with HIP events recorded on
the library's stream around that kernel in profiled calls; its `traffic` comes from the
committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary. `cpu_baseline` times the torch-CPU
restatement of the reference's decode algorithm (dense gather + bmm) on the host's cores; the
prefill object and the E=512 entries carry their own (the per-expert loop for prefill).
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = ("MoE layer µs/call + TFLOP/s (or GB/s) & % roofline, decode T=128 / "
          "prefill T=8192")
HBM_PEAK_GBS = 8000.0
SETTLE_S = 0.3      # untimed calls ahead of every configuration after the headline one
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--T", type=int, default=128)
    p.add_argument("--prefill-T", type=int, default=8192)
    p.add_argument("--shape", default="qwen3-30b-a3b")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-budget-s", type=float, default=20.0)
    p.add_argument("--no-extra", action="store_true",
                   help="skip the other configurations (decode sweep, E=512 layer, fp8 variant)")
    p.add_argument("--only-extra", default=None, metavar="TEXT",
                   help="run only the extra configurations whose name contains TEXT (for example "
                        "'fp8-e4m3 prefill') and print them as one JSON line, without the "
                        "headline measurement")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="also run a plain copy kernel (torch.neg, fp32) over this many MiB, "
                        "3 times: the calibration dispatch for FETCH_SIZE/WRITE_SIZE counters")
    return p.parse_args()


class HipEvents:
    """hipEvent_t helpers through the HIP runtime torch has loaded."""

    def __init__(self):
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64" in line:
                    path = line.split()[-1]
                    break
        self.h = ctypes.CDLL(path or "libamdhip64.so.7")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.h.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        evs = (ctypes.c_void_p * n)()
        for i in range(n):
            e = ctypes.c_void_p()
            assert self.h.hipEventCreate(ctypes.byref(e)) == 0
            evs[i] = e
        return evs

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        assert self.h.hipEventSynchronize(b) == 0
        assert self.h.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value


def layer_inputs(shape, T, seed, zipf, device, fp8=False):
    import torch
    from layerbatch_amd.moe import Qwen3_5SparseMoeBlock
    from layerbatch_amd.synth import make_layer, make_x, zipf_bias
    w, g = make_layer(shape, seed=seed, device=device)
    x = make_x(g, T, shape.hidden_size, device=device)
    blk = Qwen3_5SparseMoeBlock(shape.hidden_size, shape.num_experts, shape.top_k,
                                shape.moe_intermediate_size, shape.shared_expert_intermediate_size)
    blk = blk.to(device=device, dtype=torch.bfloat16)
    with torch.no_grad():
        blk.gate.weight.copy_(w["gate"])
        blk.experts.gate_up_proj.copy_(w["gate_up"])
        blk.experts.down_proj.copy_(w["down"])
        if shape.shared_expert_intermediate_size:
            blk.shared_expert.gate_proj.weight.copy_(w["sh_gate"])
            blk.shared_expert.up_proj.weight.copy_(w["sh_up"])
            blk.shared_expert.down_proj.weight.copy_(w["sh_down"])
            blk.shared_expert_gate.weight.copy_(w["sh_gate_w"])
    if zipf:
        blk.gate.logit_bias = zipf_bias(g, shape.num_experts, device=device)
    if fp8:
        blk.quantize_fp8_()
    del w
    return blk, x


def settle(call, warmup, settle_s):
    """`warmup` untimed calls, then more until `settle_s` seconds of calls have run: the GPU's
    clocks take tens of milliseconds of sustained work to ramp up from idle (a prefill call
    runs ~25% slower over its first ~30 calls), so a configuration measured right after
    another phase of the run (allocation, host work) is timed in its steady state."""
    import torch
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < settle_s:
        for _ in range(4):
            call()
        torch.cuda.synchronize()


def check_all(rcs, what="lbmoe_forward"):
    """Status of every timed call, checked once the timed region has ended: a failed call
    invalidates the measurement."""
    from layerbatch_amd import _lib
    for rc in rcs:
        _lib.check(rc, what)


# Timed calls of every prefill-sized measurement, whatever --steps is (one call is ~1 ms).
MIN_PREFILL_STEPS = 10


def measure(blk, x, steps, warmup, hip, settle_s=0.0):
    """Wall time per call over `steps` plain calls, then per-stage HIP-event times over
    `steps` profiled calls. Returns a dict of timings and routing statistics."""
    import torch
    from layerbatch_amd import _lib
    T = x.shape[0]
    L = blk.layer()
    ws = torch.empty(_lib.workspace_size(L, T), dtype=torch.uint8, device=x.device)
    y = torch.empty_like(x)
    lib = _lib.lib()
    stream = _lib.stream_of(x.device)
    args = (ctypes.byref(L), _lib.ptr(x), T, _lib.ptr(y), _lib.ptr(ws), ws.numel(), stream)
    settle(lambda: _lib.check(lib.lbmoe_forward(*args), "lbmoe_forward"), warmup, settle_s)
    t0 = time.perf_counter()
    rcs = [lib.lbmoe_forward(*args) for _ in range(steps)]
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - t0) / steps * 1e6
    check_all(rcs)

    n_ev = _lib.LBMOE_PROFILE_EVENTS
    evsets = [hip.create(n_ev) for _ in range(steps)]
    torch.cuda.synchronize()
    for evs in evsets:
        _lib.check(lib.lbmoe_forward_profiled(*args, evs, n_ev), "lbmoe_forward_profiled")
    torch.cuda.synchronize()
    stages = {name: 0.0 for name in _lib.PROFILE_STAGES}
    for evs in evsets:
        for i, name in enumerate(_lib.PROFILE_STAGES):
            stages[name] += hip.elapsed_ms(evs[i], evs[i + 1]) * 1e3 / steps
    off, nb = _lib.workspace_region(L, T, "counts")
    counts = ws[off:off + 4 * blk.gate.num_experts].view(torch.int32).cpu()
    return {"wall_us": wall_us, "stage_us": stages, "hit_experts": int((counts > 0).sum()),
            "max_tokens_per_expert": int(counts.max()), "y": y}


def work(shape, T, n_hit, wb=2):
    """Algorithmic bytes/flops of the layer and of its gate_up kernel (wb: bytes per expert
    weight element; fp8 adds its per-128x128-block fp32 scales)."""
    H, E, k, I, Is = (shape.hidden_size, shape.num_experts, shape.top_k,
                      shape.moe_intermediate_size, shape.shared_expert_intermediate_size)
    sc = 3 * (H // 128) * (I // 128) * 4 if wb == 1 else 0      # scale bytes per expert
    scs = 3 * (H // 128) * (Is // 128) * 4 if wb == 1 and Is else 0
    layer_bytes = (n_hit * (3 * H * I * wb + sc) + (3 * H * Is * wb + scs + H * 2 if Is else 0)
                   + E * H * 2 + 2 * T * H * 2)
    layer_flops = 2 * T * k * 3 * H * I + 2 * T * 3 * H * Is + 2 * T * E * H
    gu_bytes = n_hit * 2 * I * H * wb + (2 * Is * H * wb if Is else 0) + T * H * 2 + (T * k * I + (T * Is if Is else 0)) * 2
    gu_flops = 2 * T * k * 2 * H * I + 2 * T * 2 * H * Is
    return layer_bytes, layer_flops, gu_bytes, gu_flops


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "moe_decode_qwen3-30b-a3b_T128_pmc_traffic.txt")
PREFILL_TRAFFIC_FILE = os.path.join(ROOT, "profiles",
                                    "moe_prefill_qwen3-30b-a3b_T8192_zipf_pmc_traffic.txt")


def pmc_traffic(kernel, path=TRAFFIC_FILE):
    """HBM bytes per dispatch of `kernel` at the default workload, from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (calibrated against a copy kernel); None if the summary is
    absent."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(kernel) and line[len(kernel)] in " <":
                    return int(line.split()[-1])
    except OSError:
        pass
    return None


def cpu_baseline(blk, x, zipf, budget_s):
    """The torch-CPU restatement of the reference path on this host's cores: the algorithm the
    reference picks for this batch (dense gather + bmm for decode, the per-expert loop for
    prefill, qwen3_5.py:808-813), shared expert included, on the block's bf16 weights (a block
    converted to fp8 keeps them; the reference has no fp8 path). One warmup, then the median of
    up to 5 calls within budget_s."""
    import torch
    from oracle import torch_ref
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)

    def cpu(t):
        return None if t is None else t.detach().cpu()

    wg = cpu(blk.gate.weight)
    wgu = cpu(blk.experts.gate_up_proj)
    wd = cpu(blk.experts.down_proj)
    sh = None
    if blk.shared_expert is not None:
        se = blk.shared_expert
        sh = (cpu(se.gate_proj.weight), cpu(se.up_proj.weight), cpu(se.down_proj.weight),
              cpu(blk.shared_expert_gate.weight))
    bias = cpu(blk.gate.logit_bias)
    xc = x.cpu()
    algorithm = "sparse" if zipf or x.shape[0] > 512 else "dense"
    k = blk.gate.top_k
    times = []
    with torch.inference_mode():
        t0 = time.perf_counter()
        torch_ref.block(xc, wg, wgu, wd, k, bias=bias, sh=sh, algorithm=algorithm)   # warmup
        first = time.perf_counter() - t0
        n = max(1, min(5, int(budget_s / max(first, 1e-3))))
        for _ in range(n):
            t0 = time.perf_counter()
            torch_ref.block(xc, wg, wgu, wd, k, bias=bias, sh=sh, algorithm=algorithm)
            times.append(time.perf_counter() - t0)
    times.sort()
    return {"us_per_call": times[len(times) // 2] * 1e6, "cores": ncores, "calls": len(times),
            "algorithm": algorithm}


def cpu_entry(c, value, unit, what):
    """cpu_baseline object of the JSON line from a cpu_baseline() result."""
    return {"value": value, "unit": unit, "cores": c["cores"], "kind": "port",
            "us_per_call": round(c["us_per_call"], 1),
            "sample": f"{c['calls']} timed calls (median, after 1 warmup) of the torch-CPU "
                      f"restatement of the reference's {c['algorithm']} algorithm, {what}"}


def measure_wall(blks, x, steps, warmup):
    """Back-to-back lbmoe_forward calls cycling over `blks` (copies of one layer, so that the
    weights touched per call exceed the 256 MB MALL); returns (us per call, experts hit)."""
    import torch
    from layerbatch_amd import _lib
    T = x.shape[0]
    lib = _lib.lib()
    stream = _lib.stream_of(x.device)
    y = torch.empty_like(x)
    calls = []
    for blk in blks:
        L = blk.layer()
        ws = torch.empty(_lib.workspace_size(L, T), dtype=torch.uint8, device=x.device)
        calls.append((L, ws, (ctypes.byref(L), _lib.ptr(x), T, _lib.ptr(y), _lib.ptr(ws),
                              ws.numel(), stream)))
    it = iter(range(1 << 62))
    settle(lambda: _lib.check(lib.lbmoe_forward(*calls[next(it) % len(calls)][2]), "lbmoe_forward"),
           warmup, SETTLE_S)
    t0 = time.perf_counter()
    rcs = [lib.lbmoe_forward(*calls[i % len(calls)][2]) for i in range(steps)]
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / steps * 1e6
    check_all(rcs)
    L, ws, _ = calls[0]
    off, _ = _lib.workspace_region(L, T, "counts")
    counts = ws[off:off + 4 * L.num_experts].view(torch.int32).cpu()
    return us, int((counts > 0).sum())


def norm_config(name, shape, hid, res, nw, steps, dev, eps=1e-6):
    """Back-to-back µs per call of the block with the decoder layer's residual add + RMSNorm:
    fused (lbmoe_forward_norm), the block alone on an already normalised input, and the
    reference's torch statements for the add and the norm followed by the block."""
    import torch
    from layerbatch_amd import _lib
    T = hid.shape[0]
    blk, _ = layer_inputs(shape, 1, 0, False, dev)
    L = blk.layer()
    lib = _lib.lib()
    stream = _lib.stream_of(dev)
    ws = torch.empty(_lib.workspace_size(L, T), dtype=torch.uint8, device=dev)
    y = torch.empty_like(hid)
    new_res = torch.empty_like(res)
    xn = torch.empty_like(hid)
    fused = (ctypes.byref(L), _lib.ptr(hid), _lib.ptr(res), _lib.ptr(nw), eps, T, _lib.ptr(y),
             _lib.ptr(new_res), _lib.ptr(ws), ws.numel(), stream)
    plain = (ctypes.byref(L), _lib.ptr(xn), T, _lib.ptr(y), _lib.ptr(ws), ws.numel(), stream)

    def torch_norm():
        h = res + hid                                     # qwen3_5.py:998
        o = h.float()                                     # Qwen3_5RMSNorm, :48-55
        o = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + eps)
        xn.copy_((o * (1.0 + nw.float())).type_as(h))

    def timed(fn):
        settle(fn, max(2, steps // 5), SETTLE_S)
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps * 1e6

    torch_norm()
    us_fused = timed(lambda: _lib.check(lib.lbmoe_forward_norm(*fused), "lbmoe_forward_norm"))
    us_plain = timed(lambda: _lib.check(lib.lbmoe_forward(*plain), "lbmoe_forward"))
    us_torch = timed(lambda: (torch_norm(), _lib.check(lib.lbmoe_forward(*plain), "lbmoe_forward")))
    del blk
    return {"config": name, "T": T, "us_per_call_fused": round(us_fused, 1),
            "us_per_call_block_only": round(us_plain, 1),
            "us_per_call_torch_norm_then_block": round(us_torch, 1), "bound": "hbm"}


def extra_configs(dev, steps, only=None, cpu_budget_s=0.0):
    """The other configurations of the measurement plan, each at one GPU: the decode sweep of
    the headline layer, the Qwen3-Next-style E=512 layer with a shared expert, and its fp8
    variant. Every entry: back-to-back us per call and the algorithmic rate. only: run just
    the configurations whose name contains this text."""
    import torch
    from layerbatch_amd.synth import SHAPES, make_x
    out = []

    def entry(name, shape, T, us, hit, wb, bound):
        lb, lf, _, _ = work(shape, T, hit, wb)
        gbs = lb / (us * 1e-6) / 1e9
        tf = lf / (us * 1e-6) / 1e12
        peak_tf = FP8_PEAK_TFLOPS if wb == 1 else BF16_PEAK_TFLOPS
        return {"config": name, "T": T, "us_per_call": round(us, 1), "hit_experts": hit,
                "GBps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                "TFLOPs": round(tf, 2), "frac_of_mfma_peak": round(tf / peak_tf, 4),
                "bound": bound}

    def wanted(name):
        return only is None or only in name

    g = torch.Generator(device=dev)
    g.manual_seed(7)
    # decode sweep of the headline layer; four weight copies rotate when a call touches few
    # experts, so the weights do not stay in the 256 MB MALL between calls
    shape = SHAPES["qwen3-30b-a3b"]
    sweep = [(T, "qwen3-30b-a3b decode" + (" (4 weight copies rotating)" if T <= 16 else ""))
             for T in (1, 16, 64, 256)]
    # the activations are drawn for every configuration, so that each one sees the same inputs
    # whichever are selected
    copies = None
    if any(wanted(name) for _, name in sweep):
        copies = [layer_inputs(shape, 1, i, False, dev)[0] for i in range(4)]
    for T, name in sweep:
        x = make_x(g, T, shape.hidden_size, device=dev)
        if wanted(name):
            blks = copies if T <= 16 else copies[:1]
            us, hit = measure_wall(blks, x, steps, max(2, steps // 5))
            out.append(entry(name, shape, T, us, hit, 2, "hbm"))
        del x
    del copies
    torch.cuda.empty_cache()

    # the decoder layer's residual add + RMSNorm ahead of the block (qwen3_5.py:998-1004):
    # lbmoe_forward_norm against lbmoe_forward on the normalised input, and against the
    # reference's torch statements for the add and the norm followed by lbmoe_forward
    name = "qwen3-30b-a3b decode + residual add + RMSNorm"
    hid = make_x(g, 128, shape.hidden_size, device=dev)
    res = make_x(g, 128, shape.hidden_size, device=dev)
    nw = (make_x(g, 1, shape.hidden_size, device=dev)[0].float() * 0.1).to(torch.bfloat16)
    if wanted(name):
        out.append(norm_config(name, shape, hid, res, nw, steps, dev))
    del hid, res, nw

    shape = SHAPES["qwen3-next-e512"]
    for fp8 in (False, True):
        runs = [(T, "qwen3-next-e512" + (" fp8-e4m3" if fp8 else "") +
                 (" prefill" if T > 256 else " decode"))
                for T in ((128, 16384) if fp8 else (128, 4096))]
        blk = (layer_inputs(shape, 1, 0, False, dev, fp8=fp8)[0]
               if any(wanted(name) for _, name in runs) else None)
        for T, name in runs:
            x = make_x(g, T, shape.hidden_size, device=dev)
            if wanted(name):
                n = steps if T <= 256 else max(MIN_PREFILL_STEPS, steps // 5)
                us, hit = measure_wall([blk], x, n, max(1, n // 5))
                e = entry(name, shape, T, us, hit, 1 if fp8 else 2,
                          "mfma" if fp8 and T > 256 else "hbm")
                if cpu_budget_s > 0:
                    # the reference has no fp8 path: its bf16 path on the same layer instead
                    c = cpu_baseline(blk, x, False, cpu_budget_s)
                    lb, lf, _, _ = work(shape, T, hit, 2)
                    what = (f"the bf16 layer these fp8 weights were quantised from (the "
                            f"reference has no fp8 path), T={T}, same inputs" if fp8 else
                            f"the whole layer at the same T={T} on the same inputs")
                    e["cpu_baseline"] = (cpu_entry(c, round(lf / (c["us_per_call"] * 1e-6) / 1e12, 4),
                                                   "TFLOP/s", what) if T > 256 else
                                         cpu_entry(c, round(lb / (c["us_per_call"] * 1e-6) / 1e9, 3),
                                                   "GB/s", what))
                out.append(e)
            del x
        del blk
        torch.cuda.empty_cache()
    return out



def copy_probe(mib, dev):
    """A plain copy kernel (torch.neg, fp32) over `mib` MiB, 3 times: the calibration dispatch
    for the FETCH_SIZE / WRITE_SIZE counters (reads and writes `mib` MiB each)."""
    if not mib:
        return
    import torch
    src = torch.ones(mib << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (got --gpus {args.gpus}); the MoE layer is "
              "measured at one GPU's share and no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)
    import torch
    from layerbatch_amd.synth import SHAPES
    dev = torch.device("cuda:0")
    if args.only_extra is not None:
        extra = extra_configs(dev, args.steps, args.only_extra)
        copy_probe(args.copy_probe_mib, dev)
        print(json.dumps({"metric": METRIC, "extra": extra}))
        return
    hip = HipEvents()
    shape = SHAPES[args.shape]

    blk, x = layer_inputs(shape, args.T, 0, False, dev)
    d = measure(blk, x, args.steps, args.warmup, hip)
    lb, lf, gb, gf = work(shape, args.T, d["hit_experts"])
    gu_us = d["stage_us"]["gate_up"]
    gu_gbs = gb / (gu_us * 1e-6) / 1e9
    layer_gbs = lb / (d["wall_us"] * 1e-6) / 1e9

    cpu = None
    if not args.no_cpu_baseline:
        c = cpu_baseline(blk, x, False, args.cpu_budget_s)
        cpu = cpu_entry(c, round(lb / (c["us_per_call"] * 1e-6) / 1e9, 3), "GB/s",
                        f"the whole layer at the same T={args.T} on the same inputs")
    del blk, x
    torch.cuda.empty_cache()

    prefill = None
    if not args.no_prefill:
        default_prefill = args.shape == "qwen3-30b-a3b" and args.prefill_T == 8192
        pblk, px = layer_inputs(shape, args.prefill_T, 0, True, dev)
        steps = max(MIN_PREFILL_STEPS, args.steps // 5)
        p = measure(pblk, px, steps, max(1, args.warmup // 5), hip, SETTLE_S)
        plb, plf, pgb, pgf = work(shape, args.prefill_T, p["hit_experts"])
        pgu = p["stage_us"]["gate_up"]
        prefill = {
            "T": args.prefill_T, "router_bias": "zipf(1.2)", "us_per_call": round(p["wall_us"], 1),
            "tflops": round(plf / (p["wall_us"] * 1e-6) / 1e12, 2),
            "frac_of_bf16_mfma_peak": round(plf / (p["wall_us"] * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "hit_experts": p["hit_experts"], "max_tokens_per_expert": p["max_tokens_per_expert"],
            "stage_us": {k_: round(v, 1) for k_, v in p["stage_us"].items()},
            "gate_up_tflops": round(pgf / (pgu * 1e-6) / 1e12, 2),
            "roofline": {"kernel": "tiled_persistent_kernel<kGateUp>", "bound": "mfma",
                         "achieved": round(pgf / (pgu * 1e-6) / 1e12, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s",
                         "frac": round(pgf / (pgu * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                         "algorithmic_flops_per_launch": pgf, "avg_launch_us": round(pgu, 1),
                         "traffic": (pmc_traffic("tiled_persistent_kernel<1>", PREFILL_TRAFFIC_FILE)
                                     if default_prefill else None)},
            "cpu_baseline": None,
        }
        if not args.no_cpu_baseline:
            c = cpu_baseline(pblk, px, True, args.cpu_budget_s)
            prefill["cpu_baseline"] = cpu_entry(
                c, round(plf / (c["us_per_call"] * 1e-6) / 1e12, 4), "TFLOP/s",
                f"the whole layer at the same T={args.prefill_T} with the same Zipf(1.2) router "
                f"bias on the same inputs")
        del pblk, px

    extra = None if args.no_extra else extra_configs(
        dev, args.steps, cpu_budget_s=0.0 if args.no_cpu_baseline else args.cpu_budget_s / 2)

    copy_probe(args.copy_probe_mib, dev)

    default_workload = args.shape == "qwen3-30b-a3b" and args.T == 128
    # the decode gate_up kernel at T=128 (which also derives its expert's rows from the route)
    traffic = pmc_traffic("gate_up_bf16_perm_kernel") if default_workload else None

    out = {
        "metric": METRIC, "value": round(layer_gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(d["wall_us"] / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seed 0, weights ~N(0,0.02), activations ~N(0,1), random init)",
        "config": {"workload": f"{args.shape} MoE layer decode", "hidden_size": shape.hidden_size,
                   "num_experts": shape.num_experts, "top_k": shape.top_k,
                   "moe_intermediate_size": shape.moe_intermediate_size,
                   "shared_expert_intermediate_size": shape.shared_expert_intermediate_size,
                   "T": args.T, "weights": "bf16"},
        "us_per_call": round(d["wall_us"], 2),
        "layer_frac_of_hbm_peak": round(layer_gbs / HBM_PEAK_GBS, 4),
        "hit_experts": d["hit_experts"],
        "stage_us": {k_: round(v, 2) for k_, v in d["stage_us"].items()},
        "stage_note": ("stage_us: HIP events between the stages of lbmoe_forward_profiled calls "
                       "(one call at a time); us_per_call: back-to-back lbmoe_forward calls, which "
                       "run under the sustained power limit and so slower per stage"),
        "roofline": {"kernel": "gate_up_bf16_perm_kernel", "bound": "hbm", "achieved": round(gu_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": gb,
                     "avg_launch_us": round(gu_us, 2)},
        "cpu_baseline": cpu,
        "prefill": prefill,
        "extra": extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
