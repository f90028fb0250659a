"""Benchmark of the MI355X QLoRA NF4 hot path (one JSON line on stdout).

Workload (the configuration its metric is quoted on):
one Qwen2.5-1.5B decoder layer's seven NF4 projections (q 1536->1536 +bias,
k/v 1536->256 +bias, o 1536->1536, gate/up 1536->8960, down 8960->1536), each
with a LoRA adapter r=16, alpha=32, fp16; a step is the forward of all seven
on a packed batch of T tokens (4 rows, lengths uniform in [80, 400], seed 0)
followed by their backward (dX, dA, dB).  Inputs are seeded synthetic tensors
already resident in HBM.

value      = algorithmic TFLOP/s of the whole step (base fwd + dX, LoRA fwd/bwd)
ms_per_step = the layer's fwd+bwd time (the metric's "QLoRA layer fwd+bwd ms"):
             the step is captured once as a HIP graph and replayed K times
             (same kernels, same work; no per-launch host cost).
             eager_ms_per_step is the same step launched from Python.
roofline   = the dominant NF4 entry point's achieved TFLOP/s (algorithmic
             flops per call / average call duration from HIP events recorded on
             its launch stream around every call of eager steps queued behind
             a GPU spin, so the calls run back to back as in the graph; ROCm
             does not allow timing event nodes inside a captured graph)
             against the MI355X dense fp16 MFMA peak
cpu_baseline = the oracle's "dequantize then fp32 BLAS matmul" port of the
             same step (oracle/baseline.py) timed on this host's cores
full_decoder_layer = the whole decoder layer (norms, seven QLoRA projections, RoPE,
             packed causal attention, SwiGLU, residual adds) fwd+bwd on the same
             batch, HIP-graph replay (the north star's full-layer time)
other_configs = configs[0] (gate dequant GB/s, GEMM T=1024 TFLOP/s), configs[2]
             (add-RMSNorm fwd/bwd/bwd+dgamma and unpad gather/scatter GB/s),
             configs[3] (fused chunked CE fwd+bwd ms and TFLOP/s), and the
             configs[1] layer's MLP activation: SwiGLU fwd/bwd GB/s and the frozen
             NF4 MLP fwd+bwd with the SwiGLU in the GEMM epilogues or as its own
             kernels
sweep_configs4 = configs[4]: NF4 forward and dX at the Qwen2.5-7B projection
             shapes, T in {1, 16, 128, 2048, 16384}, each point timed from HBM
             (GB/s, TFLOP/s, fraction of its HBM or MFMA roofline)
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-graph]
       [--no-sweep] [--no-full-layer] [--no-other-configs]
"""

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = ("NF4-GEMM TFLOP/s & HBM GB/s (Qwen2.5-1.5B shapes); QLoRA layer fwd+bwd ms")
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA (AMD published)
PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-graph", action="store_true",
                   help="time eager steps instead of HIP-graph replays of the step")
    p.add_argument("--timing-steps", type=int, default=5,
                   help="eager steps (queued behind a GPU spin) whose per-call HIP events "
                        "give the roofline kernel timing")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-sweep", action="store_true",
                   help="skip the configs[4] NF4 GEMM sweep (7B shapes, T in {1,16,128,2048,16384})")
    p.add_argument("--no-full-layer", action="store_true",
                   help="skip the whole-decoder-layer timing (full_decoder_layer: null)")
    p.add_argument("--no-other-configs", action="store_true",
                   help="skip configs[0], configs[2] and configs[3] (dequant, GEMM T=1024, "
                        "add-RMSNorm, unpad, fused CE)")
    p.add_argument("--profile-call", default="", metavar="DIR:N:K",
                   help="only run one configs[1] projection entry point (DIR forward or "
                        "backward, weight [N,K]) --reps times at the bench's T and exit (for "
                        "rocprofv3 counter passes that attribute every kernel to one call)")
    p.add_argument("--profile-mlp", action="store_true",
                   help="only run the configs[1] layer's frozen NF4 MLP forward + backward "
                        "(SwiGLU as its own kernels) --reps times at the bench's T and exit")
    p.add_argument("--profile-sweep", default="", metavar="NAME:T:MODE",
                   help="only run one configs[4] point (NAME in q_o, k_v, gate_up, down; MODE "
                        "fwd or dx) --reps times, rotating weight copies as the sweep does, "
                        "and exit (for rocprofv3 kernel-trace and counter passes)")
    p.add_argument("--profile-layer", action="store_true",
                   help="only run the full decoder layer (layer.DecoderLayer) forward + backward "
                        "--reps times on the configs[1] batch and exit (for a kernel trace)")
    p.add_argument("--profile-ce", action="store_true",
                   help="only run the configs[3] fused CE forward + backward --reps times and "
                        "exit (for a rocprofv3 kernel trace)")
    p.add_argument("--profile-read", default="", metavar="NAME",
                   help="only run the HBM read probe over the codes of one configs[4] weight "
                        "(NAME as in --profile-sweep) --reps times with --read-blocks "
                        "workgroups, rotating copies, and exit (for a rocprofv3 kernel trace)")
    p.add_argument("--read-blocks", type=int, default=1024)
    p.add_argument("--reps", type=int, default=20)
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run 10 device-to-device copies of MIB MiB (scales rocprofv3 "
                        "FETCH_SIZE / WRITE_SIZE to bytes) and exit")
    return p.parse_args()


def copy_calibration(mib):
    """Plain copy kernel of known size: each dispatch reads and writes exactly mib MiB."""
    import torch

    n = mib << 20
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    print(json.dumps({"copy_calibration_bytes_per_dispatch": n, "dispatches": 10}), flush=True)


def profile_mlp(reps):
    """Repeat the frozen NF4 MLP step (gate/up 8960x1536, down 1536x8960) of the layer."""
    import torch

    from soupsuck_amd import mlp as fmlp
    from soupsuck_amd.bnb_compat import quantize_4bit

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    tokens, h, inter = sum(lengths_config1()), 1536, 8960
    parts = []
    for n, k in ((inter, h), (inter, h), (h, inter)):
        packed, st = quantize_4bit((torch.randn((n, k), device=dev, generator=gen) * 0.02).half())
        parts.append((packed, st, n, k))
    x = torch.randn((tokens, h), device=dev, generator=gen).half()
    g = torch.randn((tokens, h), device=dev, generator=gen).half()
    torch.cuda.synchronize()
    for _ in range(reps):
        _, gate, up = fmlp.mlp_forward_2d(x, parts, keep=True)
        fmlp.mlp_backward_2d(g, parts, gate, up)
    torch.cuda.synchronize()
    print(json.dumps({"profile_mlp": True, "tokens": tokens, "reps": reps}), flush=True)


def profile_call(spec, reps):
    """Repeat one ss_qlora_forward / ss_qlora_backward call of the configs[1] layer."""
    import torch

    from soupsuck_amd import _lib
    from soupsuck_amd.layer import QLoRALayer

    direction, n, k = spec.split(":")
    n, k = int(n), int(k)
    device = torch.device("cuda:0")
    layer = QLoRALayer(device)
    tokens = sum(lengths_config1())
    xs, gs = layer.inputs(tokens, device)
    idx = next(i for i, p in enumerate(layer.projections) if (p.n, p.k) == (n, k))
    proj, x, g = layer.projections[idx], xs[idx], gs[idx]
    from soupsuck_amd.lora import qlora_projection

    x.requires_grad_(direction == "backward")
    out = qlora_projection(x, proj.lora_a, proj.lora_b, proj.packed, proj.state, proj.bias,
                           layer.scaling)
    torch.cuda.synchronize()
    for _ in range(reps):
        if direction == "backward":
            out.backward(g, retain_graph=True)
        else:
            qlora_projection(x, proj.lora_a, proj.lora_b, proj.packed, proj.state, proj.bias,
                             layer.scaling)
    torch.cuda.synchronize()
    print(json.dumps({"profile_call": spec, "tokens": tokens, "reps": reps}), flush=True)


def measured_traffic():
    """HBM bytes per entry-point call from the committed rocprofv3 --pmc summaries
    (FETCH_SIZE and WRITE_SIZE passes, each scaled by a copy kernel of known size)."""
    found = {}
    for path in sorted((ROOT / "profiles").glob("*.md")):
        for line in path.read_text().splitlines():
            if line.startswith("traffic-json:"):
                for key, val in json.loads(line.split(":", 1)[1]).items():
                    found[key] = (val["traffic_bytes"], path.name)
    return found


TIMED_ENTRY_POINTS = ("ss_nf4_gemm_fwd", "ss_nf4_gemm_dx", "ss_qlora_fwd", "ss_qlora_dx",
                      "ss_qlora_forward", "ss_qlora_backward")

# Rank-16 LoRA flops an entry point performs besides the base 2*T*N*K:
# forward Z = X.A^T and Z.B^T; backward dZ, dB, dA and dZ.A.
LORA_FLOPS = {"ss_qlora_forward": lambda t, n, k: 2 * t * 16 * (k + n),
              "ss_qlora_backward": lambda t, n, k: 2 * t * 16 * (2 * n + 2 * k)}


def sleep_cycles_per_ms(torch):
    """Clock rate of torch.cuda._sleep's spin loop, measured with HIP events."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1000)
    start.record()
    torch.cuda._sleep(2_000_000)
    end.record()
    end.synchronize()
    return 2_000_000 / max(start.elapsed_time(end), 1e-3)


def lengths_config1():
    import torch

    gen = torch.Generator(device="cpu").manual_seed(0)
    return [int(v) for v in torch.randint(80, 401, (4,), generator=gen)]


class KernelTimer:
    """HIP events around every NF4 GEMM entry point call, on its launch stream (torch's
    current stream), keyed by entry point and shape.  One call is one launch sequence
    (e.g. the QLoRA backward: the preparation launch with dZ, dB and the transposed
    decode, the MFMA GEMM, then dA)."""

    def __init__(self):
        import torch

        self.torch = torch
        self.records = []
        self.active = False
        self._pending = None

    def _event(self):
        return self.torch.cuda.Event(enable_timing=True)

    def before(self, name, args):
        if not self.active:
            return
        start = self._event()
        start.record()
        self._pending = (name, args, start)

    def after(self, name, args):
        if not self.active or self._pending is None:
            return
        end = self._event()
        end.record()
        _, a, start = self._pending
        self._pending = None
        t, n, k = a[2], a[8], a[9]
        flops = 2.0 * t * n * k + LORA_FLOPS.get(name, lambda *_: 0)(t, n, k)
        self.records.append((f"{name}[T={t},N={n},K={k}]", flops, start, end))

    def summary(self):
        per = {}
        for key, flops, start, end in self.records:
            ms = start.elapsed_time(end)
            agg = per.setdefault(key, [0, 0.0, 0.0])
            agg[0] += 1
            agg[1] += flops
            agg[2] += ms
        return {k: {"launches": v[0], "avg_us": 1e3 * v[2] / v[0],
                    "avg_gflop": v[1] / v[0] / 1e9,
                    "tflops": v[1] / (v[2] * 1e-3) / 1e12,
                    "total_ms": v[2]} for k, v in per.items()}


# Qwen2.5-7B projection shapes (hidden 3584, intermediate 18944,
# kv 512) as (name, N, K) of W [N, K]; T values of the sweep.
SWEEP_SHAPES = [("q_o", 3584, 3584), ("k_v", 512, 3584), ("gate_up", 18944, 3584),
                ("down", 3584, 18944)]
SWEEP_T = [1, 16, 128, 2048, 16384]


def sweep_weight(torch, name, n, k, gen, dev):
    """Quantized weight of one configs[4] shape and enough copies of its codes and
    block scales (> 300 MB in total) that rotating over them reads HBM, not the
    256 MB last-level cache."""
    from soupsuck_amd.bnb_compat import quantize_4bit

    w = (torch.randn((n, k), device=dev, generator=gen) * 0.02).half()
    packed, st = quantize_4bit(w)
    del w
    wbytes = n * k // 2 + n * k // 64 + 4 * ((n * k // 64 + 255) // 256)
    copies = max(1, -(-300_000_000 // wbytes))
    states = [(packed.clone(), st.absmax.clone()) for _ in range(copies)]
    rest = (st.state2.absmax.data_ptr(), st.state2.code.data_ptr(), st.offset.data_ptr())
    return {"states": states, "rest": rest, "copies": copies, "wbytes": wbytes, "keep": st}


def sweep_call(torch, _lib, weight, n, k, t, mode, gen, dev):
    """call(i, stream) of one configs[4] point (weight copy i % copies) and its buffers."""
    lib = _lib.load()
    size = lib.ss_nf4_gemm_workspace_size(t, n, k)
    ws = torch.empty(max(size, 16), device=dev, dtype=torch.uint8)
    a = torch.randn((t, n if mode == "dx" else k), device=dev, generator=gen).half()
    o = torch.empty((t, k if mode == "dx" else n), device=dev, dtype=torch.float16)
    states, rest, copies = weight["states"], weight["rest"], weight["copies"]

    def call(i, stream):
        pk, am = states[i % copies]
        if mode == "dx":
            _lib.call("ss_nf4_gemm_dx", a.data_ptr(), a.stride(0), t, pk.data_ptr(),
                      am.data_ptr(), *rest, n, k, o.data_ptr(), o.stride(0), 0,
                      ws.data_ptr(), size, stream)
        else:
            _lib.call("ss_nf4_gemm_fwd", a.data_ptr(), a.stride(0), t, pk.data_ptr(),
                      am.data_ptr(), *rest, n, k, None, o.data_ptr(), o.stride(0),
                      ws.data_ptr(), size, stream)

    call.buffers = (ws, a, o)
    return call


def sweep(torch, _lib):
    """NF4 forward and dX at every configs[4] shape and T through the C ABI.

    Each point is the average of R calls captured in one HIP graph (no host
    launch cost), rotating over copies of the packed weight whose total
    exceeds the 256 MB last-level cache, so every call streams its weight
    from HBM.  Algorithmic bytes: packed codes + qabs + absmax2 + the fp16
    activation read and output written; flops 2*T*N*K.  roofline_frac =
    max(bytes / 8 TB/s, flops / 2.5 PFLOP/s) / measured time."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    out = {}
    for name, n, k in SWEEP_SHAPES:
        weight = sweep_weight(torch, name, n, k, gen, dev)
        for t in SWEEP_T:
            for mode in ("fwd", "dx"):
                call = sweep_call(torch, _lib, weight, n, k, t, mode, gen, dev)
                flops = 2.0 * t * n * k
                reps = max(4, min(64, int(2e10 / max(flops, 1.0))))
                us = graph_us(torch, _lib, call, reps)
                moved = weight["wbytes"] + 2 * t * (n + k)
                bound_us = max(moved / PEAK_HBM_GBS / 1e3, flops / PEAK_FP16_TFLOPS / 1e6)
                out[f"{name} T={t} {mode}"] = {
                    "N": n, "K": k, "us": round(us, 2), "GB/s": round(moved / us / 1e3, 1),
                    "TFLOP/s": round(flops / us / 1e6, 2),
                    "bound": "hbm" if moved / PEAK_HBM_GBS / 1e3 >= flops / PEAK_FP16_TFLOPS / 1e6
                    else "mfma",
                    "roofline_frac": round(bound_us / us, 4)}
                del call
        del weight
        torch.cuda.empty_cache()
    ceiling = vendor_ceiling(torch)
    out["vendor_ceiling"] = ceiling
    reads = read_ceiling(torch, _lib)
    out["hbm_read_ceiling"] = reads
    # T = 1 forward against a plain read of the same codes: how far the NF4 stream is
    # from the board's read floor (the roofline fraction is against 8 TB/s)
    for name, _, _ in SWEEP_SHAPES:
        point, floor = out.get(f"{name} T=1 fwd"), reads.get(f"{name} codes")
        if point and floor:
            point["vs_read_ceiling_time"] = round(point["us"] / floor["us"], 3)
    # T = 2048: this build's call time over hipBLASLt's time for the same product (the
    # call includes the NF4 decode; the vendor product reads fp16 weights)
    for name, _, _ in SWEEP_SHAPES:
        for mode in ("fwd", "dx"):
            ours, vendor = out.get(f"{name} T=2048 {mode}"), ceiling.get(f"{name} T=2048 {mode}")
            if ours and vendor:
                ours["vs_vendor_time"] = round(ours["us"] / vendor["us"], 3)
    return out


def vendor_ceiling(torch):
    """Same-box reference point: torch.matmul (hipBLASLt) on fp16 operands already
    in HBM, at 8192^3, at the configs[4] T=16384 gate/up and down products, at
    every configs[4] product at T=2048 and at every configs[1] projection's product
    at T=990 (the dense part of the headline step), forward X [T, K] . W^T and dX
    dY [T, N] . W with W [N, K] row-major.  Average of 10 calls between HIP events after 3
    warm-ups; a probe of what the vendor GEMM reaches on this board, not a
    target."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    res = {}
    products = [("8192^3", 8192, 8192, 8192, "fwd"),
                ("gate_up T=16384 (16384x18944x3584)", 16384, 18944, 3584, "fwd"),
                ("down T=16384 (16384x3584x18944)", 16384, 3584, 18944, "fwd")]
    for name, n, k in SWEEP_SHAPES:
        for mode in ("fwd", "dx"):
            products.append((f"{name} T=2048 {mode}", 2048, n, k, mode))
    for name, n, k in (("gate/up", 8960, 1536), ("down", 1536, 8960), ("q/o", 1536, 1536),
                       ("k/v", 256, 1536)):
        for mode in ("fwd", "dx"):
            products.append((f"configs[1] {name} T=990 {mode}", 990, n, k, mode))
    for label, m, n, k, mode in products:
        a = torch.randn((m, n if mode == "dx" else k), device=dev, generator=gen).half()
        w = torch.randn((n, k), device=dev, generator=gen).half()
        c = torch.empty((m, k if mode == "dx" else n), device=dev, dtype=torch.float16)
        b = w if mode == "dx" else w.t()
        for _ in range(3):
            torch.matmul(a, b, out=c)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            torch.matmul(a, b, out=c)
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) / 10 * 1e3
        tf = 2.0 * m * n * k / us / 1e6
        res[label] = {"us": round(us, 1), "TFLOP/s": round(tf, 1),
                      "frac_of_peak": round(tf / PEAK_FP16_TFLOPS, 4)}
        del a, w, c
    torch.cuda.empty_cache()
    return res


def profile_sweep(spec, reps):
    """Repeat one configs[4] point (eager calls through the C ABI), rotating copies."""
    import torch

    from soupsuck_amd import _lib

    name, t, mode = spec.split(":")
    t = int(t)
    n, k = next((n, k) for nm, n, k in SWEEP_SHAPES if nm == name)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    weight = sweep_weight(torch, name, n, k, gen, dev)
    call = sweep_call(torch, _lib, weight, n, k, t, mode, gen, dev)
    stream = _lib.stream(dev)
    torch.cuda.synchronize()
    for i in range(reps):
        call(i, stream)
    torch.cuda.synchronize()
    print(json.dumps({"profile_sweep": spec, "N": n, "K": k, "reps": reps,
                      "weight_copies": weight["copies"]}), flush=True)


def profile_read(name, blocks, reps):
    """Repeat the HBM read probe over one configs[4] weight's code bytes, rotating copies."""
    import torch

    from soupsuck_amd import _lib

    n, k = next((n, k) for nm, n, k in SWEEP_SHAPES if nm == name)
    dev = torch.device("cuda:0")
    nbytes = n * k // 2
    copies = max(2, -(-300_000_000 // nbytes))
    bufs = [torch.empty(nbytes, device=dev, dtype=torch.uint8).fill_(i & 0xFF)
            for i in range(copies)]
    sink = torch.empty(blocks, device=dev, dtype=torch.int32)
    stream = _lib.stream(dev)
    torch.cuda.synchronize()
    for i in range(reps):
        _lib.call("ss_hbm_read_probe", bufs[i % copies].data_ptr(), nbytes, blocks,
                  sink.data_ptr(), stream)
    torch.cuda.synchronize()
    print(json.dumps({"profile_read": name, "bytes": nbytes, "blocks": blocks, "reps": reps,
                      "copies": copies}), flush=True)


def graph_us(torch, _lib, call, reps):
    """Average µs of one call(i, stream) over reps calls captured in one HIP graph."""
    dev = torch.device("cuda:0")
    call(0, _lib.stream(dev))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        sc = _lib.stream(dev)
        for i in range(reps):
            call(i, sc)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    e1.synchronize()
    del graph
    return e0.elapsed_time(e1) / reps * 1e3


def read_ceiling(torch, _lib):
    """What a plain cold read costs on this board (ss_hbm_read_probe), at the code sizes of
    the configs[4] weights: the yardstick for the small-T NF4 kernels, which read their
    codes once.  Buffers are rotated over > 300 MB (reads come from HBM, not the 256 MB
    last-level cache); each size is timed at several grid sizes in HIP graphs and the
    fastest is reported, with the matching T = 1 forward of the sweep for comparison."""
    dev = torch.device("cuda:0")
    res = {}
    for name, n, k in SWEEP_SHAPES:
        nbytes = n * k // 2
        copies = max(2, -(-300_000_000 // nbytes))
        bufs = [torch.empty(nbytes, device=dev, dtype=torch.uint8).fill_(i & 0xFF)
                for i in range(copies)]
        best = None
        for blocks in (256, 512, 1024, 2048, 4096):
            sink = torch.empty(blocks, device=dev, dtype=torch.int32)

            def call(i, stream, blocks=blocks, sink=sink):
                _lib.call("ss_hbm_read_probe", bufs[i % copies].data_ptr(), nbytes, blocks,
                          sink.data_ptr(), stream)

            us = graph_us(torch, _lib, call, 32)
            if best is None or us < best[0]:
                best = (us, blocks)
        res[f"{name} codes"] = {"bytes": nbytes, "us": round(best[0], 2), "blocks": best[1],
                                "GB/s": round(nbytes / best[0] / 1e3, 1),
                                "frac_of_8TBs": round(nbytes / PEAK_HBM_GBS / 1e3 / best[0], 4)}
        del bufs
        torch.cuda.empty_cache()
    return res


def hbm_point(us, moved, copies):
    return {"us": round(us, 2), "bytes": int(moved), "GB/s": round(moved / us / 1e3, 1),
            "bound": "hbm", "roofline_frac": round(moved / PEAK_HBM_GBS / 1e3 / us, 4),
            "copies_rotated": copies}


def other_configs(torch, _lib):
    """BASELINE.json configs[0], configs[2] and configs[3] on the GPU.

    HBM-bound points rotate over enough copies of their operands (> 300 MB)
    that each call reads from HBM, not from the 256 MB last-level cache; each
    is the average of R calls captured in one HIP graph.  Algorithmic bytes:
      dequant      0.5 + 1/64 B per weight in (codes, qabs) + absmax2 + 2 B out;
      add-RMSNorm  fwd  r, d in, s, y out (8 H B per row) + rstd 4 B + w 2 H;
                   bwd  s, gs, gy in, dr, dd out (10 H B per row) + rstd + w;
                   bwd + dgamma: the backward's bytes + the per-wave fp32 column sums
                   written and read back + dw;
      gather       T rows read + T rows written (4 H B per token);
      scatter      T rows read + B*S rows written + the int32 inverse map.
    CE is timed whole through fused_linear_cross_entropy
    (forward, then backward with the lm_head gradient), HIP events on the
    stream around each, median of 5; flops 2 T V H forward and 2 x 2 T_valid V H
    backward (dX, dW; the backward reads the forward's kept logits, and a
    recompute, when one runs, is not counted as algorithmic work)."""
    from soupsuck_amd import unpad
    from soupsuck_amd.bnb_compat import quantize_4bit

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    out = {}
    f16 = _lib.F16

    # gate [8960, 1536], dequant alone and Y = X W^T at T = 1024.
    n, k = 8960, 1536
    w = (torch.randn((n, k), device=dev, generator=gen) * 0.02).half()
    packed, st = quantize_4bit(w)
    del w
    moved = n * k // 2 + n * k // 64 + 4 * (-(-n * k // 16384)) + 1028 + 2 * n * k
    copies = max(1, -(-300_000_000 // moved))
    packs = [(packed.clone(), st.absmax.clone()) for _ in range(copies)]
    outs = [torch.empty((n, k), device=dev, dtype=torch.float16) for _ in range(copies)]
    rest = (st.state2.absmax.data_ptr(), st.state2.code.data_ptr(), st.offset.data_ptr())

    def dequant(i, stream):
        pk, am = packs[i % copies]
        _lib.call("ss_nf4_dequant_nested", pk.data_ptr(), am.data_ptr(), *rest,
                  outs[i % copies].data_ptr(), n * k, stream)

    us = graph_us(torch, _lib, dequant, 64)
    out["configs0_dequant_gate_8960x1536"] = hbm_point(us, moved, copies)
    del outs
    t = 1024
    x = torch.randn((t, k), device=dev, generator=gen).half()
    y = torch.empty((t, n), device=dev, dtype=torch.float16)
    size = _lib.load().ss_nf4_gemm_workspace_size(t, n, k)
    ws = torch.empty(max(size, 16), device=dev, dtype=torch.uint8)

    def gemm(i, stream):
        pk, am = packs[i % copies]
        _lib.call("ss_nf4_gemm_fwd", x.data_ptr(), x.stride(0), t, pk.data_ptr(),
                  am.data_ptr(), *rest, n, k, None, y.data_ptr(), y.stride(0),
                  ws.data_ptr(), size, stream)

    us = graph_us(torch, _lib, gemm, 32)
    flops = 2.0 * t * n * k
    out["configs0_gemm_T1024_gate"] = {
        "us": round(us, 2), "TFLOP/s": round(flops / us / 1e6, 1), "bound": "mfma",
        "roofline_frac": round(flops / PEAK_FP16_TFLOPS / 1e6 / us, 4)}
    del packs, packed, st, x, y, ws

    # add-RMSNorm fwd/bwd/bwd+dgamma at T in {826, 4096, 16384}, H = 1536.
    h = 1536
    wn = (1 + 0.1 * torch.randn(h, device=dev, generator=gen)).half()
    for t in (826, 4096, 16384):
        row_fwd = 8 * h + 4
        copies = max(1, -(-300_000_000 // (t * row_fwd)))
        bufs = []
        for _ in range(copies):
            r = torch.randn((t, h), device=dev, generator=gen).half()
            d = torch.randn((t, h), device=dev, generator=gen).half()
            bufs.append((r, d, torch.empty_like(r), torch.empty_like(r),
                         torch.empty(t, device=dev, dtype=torch.float32)))

        def fwd(i, stream):
            r, d, s, yy, rstd = bufs[i % copies]
            _lib.call("ss_add_rmsnorm_fwd", r.data_ptr(), f16, d.data_ptr(), f16, wn.data_ptr(),
                      f16, 1, s.data_ptr(), f16, yy.data_ptr(), f16, rstd.data_ptr(), t, h,
                      1e-6, stream)

        us = graph_us(torch, _lib, fwd, 32)
        out[f"configs2_add_rmsnorm_fwd_T{t}"] = hbm_point(us, t * row_fwd + 2 * h, copies)

        def norm_fwd(i, stream):
            r, _, _, yy, rstd = bufs[i % copies]
            _lib.call("ss_rmsnorm_fwd", r.data_ptr(), f16, h, wn.data_ptr(), f16, 1,
                      yy.data_ptr(), f16, rstd.data_ptr(), t, h, 1e-6, stream)

        # Standalone RMSNorm (x in, y out: 4 H B per row + rstd + w).
        out[f"rmsnorm_fwd_T{t}"] = hbm_point(graph_us(torch, _lib, norm_fwd, 32),
                                             t * (4 * h + 4) + 2 * h, copies)
        # Backward reuses the buffers: r -> gs, d -> gy (inputs), and writes
        # dr, dd into two fresh planes per copy.
        grads = [(torch.empty_like(b[0]), torch.empty_like(b[0])) for b in bufs]

        def bwd(i, stream):
            gs, gy, s, _, rstd = bufs[i % copies]
            dr, dd = grads[i % copies]
            _lib.call("ss_add_rmsnorm_bwd", s.data_ptr(), f16, wn.data_ptr(), f16, 1,
                      rstd.data_ptr(), gs.data_ptr(), f16, h, 1, gy.data_ptr(), f16, h, 1,
                      dr.data_ptr(), f16, dd.data_ptr(), f16, t, h, stream)

        us = graph_us(torch, _lib, bwd, 32)
        out[f"configs2_add_rmsnorm_bwd_T{t}"] = hbm_point(us, t * (10 * h + 4) + 2 * h, copies)
        waves = _lib.load().ss_add_rmsnorm_dgamma_waves(t)
        partial = torch.empty((waves, h), device=dev, dtype=torch.float32)
        dw = torch.empty(h, device=dev, dtype=torch.float16)

        def bwd_dgamma(i, stream):
            gs, gy, s, _, rstd = bufs[i % copies]
            dr, dd = grads[i % copies]
            _lib.call("ss_add_rmsnorm_bwd_dgamma", s.data_ptr(), f16, wn.data_ptr(), f16, 1,
                      rstd.data_ptr(), gs.data_ptr(), f16, h, 1, gy.data_ptr(), f16, h, 1,
                      dr.data_ptr(), f16, dd.data_ptr(), f16, 1, partial.data_ptr(),
                      dw.data_ptr(), f16, t, h, stream)

        us = graph_us(torch, _lib, bwd_dgamma, 32)
        out[f"configs2_add_rmsnorm_bwd_dgamma_T{t}"] = hbm_point(
            us, t * (10 * h + 4) + 2 * h + 2 * waves * h * 4 + 2 * h, copies)
        del bufs, grads

    # unpad gather/scatter of a [4, 360, 1536] fp16 batch.
    cg = torch.Generator(device="cpu").manual_seed(0)
    lengths = [int(v) for v in torch.randint(80, 361, (4,), generator=cg)]
    batch = unpad.make_batch(lengths, 360, dev)
    tokens, rows = batch.tokens, batch.rows
    inverse = batch.inverse()
    row_bytes = 2 * h
    moved_g = 2 * tokens * row_bytes + 8 * tokens
    copies = max(1, -(-300_000_000 // moved_g))
    padded = [torch.randn((rows, h), device=dev, generator=gen).half() for _ in range(copies)]
    packed_rows = [torch.empty((tokens, h), device=dev, dtype=torch.float16)
                   for _ in range(copies)]

    def gather(i, stream):
        _lib.call("ss_unpad_gather", padded[i % copies].data_ptr(), rows,
                  packed_rows[i % copies].data_ptr(), batch.indices.data_ptr(), tokens,
                  row_bytes, stream)

    us = graph_us(torch, _lib, gather, 64)
    out["configs2_unpad_gather_4x360"] = hbm_point(us, moved_g, copies)
    out["configs2_unpad_gather_4x360"].update(tokens=tokens, lengths=lengths)

    def scatter(i, stream):
        _lib.call("ss_unpad_scatter", packed_rows[i % copies].data_ptr(), tokens,
                  padded[i % copies].data_ptr(), inverse.data_ptr(), rows, row_bytes, stream)

    us = graph_us(torch, _lib, scatter, 64)
    out["configs2_unpad_scatter_4x360"] = hbm_point(
        us, tokens * row_bytes + rows * row_bytes + 4 * rows, copies)
    del padded, packed_rows

    # The MLP activation between the configs[1] gate/up and down projections:
    # SwiGLU forward (g, u in, a out: 6 B per element) and backward (g, u, da
    # in, dg, du out: 10 B) on [T, 8960] fp16, T = the configs[1] token count.
    t, inter = sum(lengths_config1()), 8960
    per = t * inter * 2
    copies = max(1, -(-300_000_000 // (5 * per)))
    planes = [[torch.randn((t, inter), device=dev, generator=gen).half() for _ in range(5)]
              for _ in range(copies)]
    mat = (f16, inter, 1)

    def swiglu_fwd(i, stream):
        g, u, _, a, _ = planes[i % copies]
        _lib.call("ss_swiglu_fwd", g.data_ptr(), *mat, u.data_ptr(), *mat, a.data_ptr(), *mat, t,
                  inter, stream)

    def swiglu_bwd(i, stream):
        g, u, da, dg, du = planes[i % copies]
        _lib.call("ss_swiglu_bwd", g.data_ptr(), *mat, u.data_ptr(), *mat, da.data_ptr(), *mat,
                  dg.data_ptr(), *mat, du.data_ptr(), *mat, t, inter, stream)

    out[f"mlp_swiglu_fwd_T{t}x{inter}"] = hbm_point(graph_us(torch, _lib, swiglu_fwd, 32),
                                                    3 * per, copies)
    out[f"mlp_swiglu_bwd_T{t}x{inter}"] = hbm_point(graph_us(torch, _lib, swiglu_bwd, 32),
                                                    5 * per, copies)
    del planes

    # RoPE of the configs[1] layer's attention: q 12 heads, k 2 heads, head_dim
    # 128 at T tokens, q / k as transposed [1, T, H, D] projection views, fp16
    # cos / sin [1, T, 128].  Bytes: q, k read and written (4 B per element)
    # plus cos and sin once.
    hq, hk, hd = 12, 2, 128
    qv = torch.randn((1, t, hq * hd), device=dev, generator=gen).half()
    kv = torch.randn((1, t, hk * hd), device=dev, generator=gen).half()
    cs = torch.randn((2, 1, t, hd), device=dev, generator=gen).half()
    yq = torch.empty((1, hq, t, hd), device=dev, dtype=torch.float16)
    yk = torch.empty((1, hk, t, hd), device=dev, dtype=torch.float16)
    qst, kst = (t * hq * hd, hd, hq * hd), (t * hk * hd, hd, hk * hd)
    cst = (t * hd, hd, t * hd, hd, 1)

    def rope_fwd(i, stream):
        _lib.call("ss_rope_fwd", qv.data_ptr(), f16, *qst, kv.data_ptr(), f16, *kst,
                  cs[0].data_ptr(), cs[1].data_ptr(), f16, *cst, yq.data_ptr(), f16,
                  yk.data_ptr(), f16, 1, hq, hk, t, hd // 2, stream)

    def rope_bwd(i, stream):
        # gradients written back in the projection views' layout (as the autograd node does)
        _lib.call("ss_rope_bwd", qv.data_ptr(), f16, *qst, 1, kv.data_ptr(), f16, *kst, 1,
                  cs[0].data_ptr(), cs[1].data_ptr(), f16, *cst, yq.data_ptr(), f16, *qst,
                  yk.data_ptr(), f16, *kst, 1, hq, hk, t, hd // 2, stream)

    moved = (hq + hk) * t * hd * 4 + 2 * t * hd * 2
    out[f"rope_fwd_T{t}"] = hbm_point(graph_us(torch, _lib, rope_fwd, 64), moved, 1)
    out[f"rope_bwd_T{t}"] = hbm_point(graph_us(torch, _lib, rope_bwd, 64), moved, 1)
    del qv, kv, cs, yq, yk

    # The frozen NF4 MLP of the configs[1] layer (gate/up 8960x1536, down
    # 1536x8960) forward + input-gradient backward at the same T, with the
    # SwiGLU in the GEMM epilogues and as its own kernels between plain GEMMs
    # (soupsuck_amd.mlp, the second is its default).  Weights stay resident
    # (as in the layer step); flops 7 x 2 T H I.
    from soupsuck_amd import mlp as fmlp

    parts = []
    for n_, k_ in ((inter, h), (inter, h), (h, inter)):
        wq = (torch.randn((n_, k_), device=dev, generator=gen) * 0.02).half()
        pk, stq = quantize_4bit(wq)
        parts.append((pk, stq, n_, k_))
        del wq
    xm = torch.randn((t, h), device=dev, generator=gen).half()
    gm = torch.randn((t, h), device=dev, generator=gen).half()

    def mlp_epilogue(i, stream):
        _, gate, up = fmlp.mlp_forward_2d(xm, parts, keep=True, fuse=True)
        fmlp.mlp_backward_2d(gm, parts, gate, up, fuse=True)

    def mlp_kernels(i, stream):
        _, gate, up = fmlp.mlp_forward_2d(xm, parts, keep=True, fuse=False)
        fmlp.mlp_backward_2d(gm, parts, gate, up, fuse=False)

    flops = fmlp.mlp_flops(t, h, inter)
    for name, fn in (("in_epilogue", mlp_epilogue), ("own_kernels", mlp_kernels)):
        us = graph_us(torch, _lib, fn, 8)
        out[f"mlp_fwd_bwd_T{t}_swiglu_{name}"] = {
            "us": round(us, 2), "TFLOP/s": round(flops / us / 1e6, 1), "bound": "mfma",
            "roofline_frac": round(flops / us / 1e6 / PEAK_FP16_TFLOPS, 4)}
    del parts, xm, gm

    # chunked fused linear CE, hidden [826, 1536], tied head [151936, 1536].
    hd, hw, labels, valid = ce_inputs(torch, gen, dev)
    t, v = hd.shape[0], hw.shape[0]
    fwd_ms, tot_ms = [], []
    for rep in range(6):
        e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        hd.grad = None
        hw.grad = None
        torch.cuda.synchronize()
        e0.record()
        mean = ce_forward(hd, hw, labels, valid)
        e1.record()
        mean.backward()
        e2.record()
        e2.synchronize()
        if rep:
            fwd_ms.append(e0.elapsed_time(e1))
            tot_ms.append(e0.elapsed_time(e2))
    fwd = statistics.median(fwd_ms)
    tot = statistics.median(tot_ms)
    f_fwd = 2.0 * t * v * h
    f_bwd = 2 * 2.0 * valid * v * h
    out["configs3_fused_ce_fwd_bwd"] = {
        "tokens": t, "valid": valid, "vocab": v, "chunk": 8192,
        "fwd_ms": round(fwd, 3), "fwd_bwd_ms": round(tot, 3),
        "fwd_TFLOP/s": round(f_fwd / fwd / 1e9, 1),
        "fwd_bwd_TFLOP/s": round((f_fwd + f_bwd) / tot / 1e9, 1),
        "bound": "mfma",
        "roofline_frac": round((f_fwd + f_bwd) / PEAK_FP16_TFLOPS / 1e9 / tot, 4),
        "timing": "HIP events on the stream (GPU clock) around the forward and the backward, "
                  "median of 5 after 1 warm-up; the backward's head-gradient gain max|g|/1024 "
                  "stays on the device (no host round trip between forward and backward)"}
    del hd, hw
    torch.cuda.empty_cache()
    return out


def full_layer(torch, lengths, steps, warmup):
    """The whole Qwen2.5-1.5B decoder layer (soupsuck_amd.layer.DecoderLayer: norms,
    seven QLoRA projections, RoPE, packed causal attention, SwiGLU, residual adds)
    forward + backward on the configs[1] batch: eager, then one HIP-graph capture
    replayed ``steps`` times between HIP events."""
    from soupsuck_amd.layer import DecoderLayer

    dev = torch.device("cuda:0")
    layer = DecoderLayer(dev, lengths)
    t = sum(lengths)
    gen = torch.Generator(device="cpu").manual_seed(3)
    h = torch.randn((t, 1536), generator=gen).half().to(dev).requires_grad_()
    g = (torch.randn((t, 1536), generator=gen) * 0.05).half().to(dev)
    for _ in range(warmup):
        layer.step(h, g)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        layer.step(h, g)
    torch.cuda.synchronize()
    eager_ms = 1e3 * (time.perf_counter() - t0) / steps
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            layer.step(h, g)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer.step(h, g)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = layer.flops()
    return {"workload": "Qwen2.5-1.5B decoder layer fwd+bwd (RMSNorm, q/k/v/o/gate/up/down "
                        "QLoRA r=16, RoPE, packed causal attention 12/2 heads, SwiGLU, residuals)",
            "tokens": t, "ms": round(ms, 4), "eager_ms": round(eager_ms, 4),
            "TFLOP/s": round(flops / ms / 1e9, 1), "gflop": round(flops / 1e9, 2),
            "timing": f"HIP-graph replay x{steps} between HIP events"}


def profile_layer(reps):
    """Repeat the full decoder layer's forward + backward (eager) on the configs[1] batch."""
    import torch

    from soupsuck_amd.layer import DecoderLayer

    dev = torch.device("cuda:0")
    lengths = lengths_config1()
    layer = DecoderLayer(dev, lengths)
    gen = torch.Generator(device="cpu").manual_seed(3)
    h = torch.randn((sum(lengths), 1536), generator=gen).half().to(dev).requires_grad_()
    g = (torch.randn((sum(lengths), 1536), generator=gen) * 0.05).half().to(dev)
    torch.cuda.synchronize()
    for _ in range(reps):
        layer.step(h, g)
    torch.cuda.synchronize()
    print(json.dumps({"profile_layer": True, "tokens": sum(lengths), "reps": reps}), flush=True)


def ce_inputs(torch, gen, dev):
    """hidden [826, 1536] ~ N(0,1), tied head [151936, 1536] ~ N(0, 0.02),
    labels uniform over the vocabulary with 36.5 % set to -100 (both trainable)."""
    t, v, h = 826, 151936, 1536
    hidden = torch.randn((t, h), device=dev, generator=gen).half()
    head = (torch.randn((v, h), device=dev, generator=gen) * 0.02).half()
    labels = torch.randint(0, v, (t,), device=dev, generator=gen)
    ignored = torch.rand(t, device=dev, generator=gen) < 0.365
    labels[ignored] = -100
    valid = int((labels != -100).sum().item())
    return hidden.requires_grad_(), head.requires_grad_(), labels, valid


def ce_forward(hidden, head, labels, valid):
    from soupsuck_amd.kernels.cross_entropy import fused_linear_cross_entropy

    loss, _, _, _ = fused_linear_cross_entropy(hidden, head, labels, chunk=8192, weight_grad=True)
    return loss.sum() / valid


def profile_ce(reps):
    """Repeat the configs[3] fused CE forward + backward (with the head gradient)."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    hd, hw, labels, valid = ce_inputs(torch, gen, dev)
    torch.cuda.synchronize()
    ms = []
    for _ in range(reps):
        hd.grad = None
        hw.grad = None
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        ce_forward(hd, hw, labels, valid).backward()
        e1.record()
        e1.synchronize()
        ms.append(e0.elapsed_time(e1))
    print(json.dumps({"profile_ce": True, "tokens": hd.shape[0], "valid": valid, "reps": reps,
                      "fwd_bwd_ms_median": round(statistics.median(ms[1:] or ms), 3)}),
          flush=True)


def cpu_model():
    """The host CPU's model name as lscpu reports it (else /proc/cpuinfo)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(layer, xs, gs, budget_s):
    """Time oracle/baseline.py on the host for the same step (bounded sample)."""
    import numpy as np

    from oracle import baseline, nf4 as onf4

    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()
                       if i.get("user_api") == "blas"] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    host = []
    for p, x, g in zip(layer.projections, xs, gs):
        st = p.state
        state = onf4.NF4State((p.n, p.k), p.packed.cpu().numpy().reshape(-1),
                              st.absmax.cpu().numpy(), st.state2.absmax.cpu().numpy(),
                              st.state2.code.cpu().numpy(), st.offset.cpu().numpy())
        host.append((x.detach().cpu().numpy(), state, p.lora_a.detach().cpu().numpy(),
                     p.lora_b.detach().cpu().numpy(),
                     None if p.bias is None else p.bias.cpu().numpy(), g.cpu().numpy()))
    times = []
    start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        for x, state, a, b, bias, g in host:
            baseline.projection_step(x, state, a, b, bias, g, layer.scaling)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - start >= budget_s or len(times) >= 20:
            break
    return statistics.median(times), len(times), threads


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus}, WORLD_SIZE "
              f"{world} requested); the multi-GPU sharding is a design note, not a run.",
              file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.profile_mlp:
        profile_mlp(args.reps)
        return
    if args.profile_call:
        profile_call(args.profile_call, args.reps)
        return
    if args.profile_sweep:
        profile_sweep(args.profile_sweep, args.reps)
        return
    if args.profile_read:
        profile_read(args.profile_read, args.read_blocks, args.reps)
        return
    if args.profile_ce:
        profile_ce(args.reps)
        return
    if args.profile_layer:
        profile_layer(args.reps)
        return

    import torch

    from soupsuck_amd import _lib
    from soupsuck_amd.layer import QLoRALayer

    _lib.load()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    lengths = lengths_config1()
    tokens = sum(lengths)
    layer = QLoRALayer(device)
    xs, gs = layer.inputs(tokens, device)

    def step():
        for p in layer.projections:
            p.lora_a.grad = None
            p.lora_b.grad = None
        for x in xs:
            x.grad = None
        layer.step(xs, gs)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Eager steps: every kernel launched from Python through the C ABI.
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_ms = 1e3 * (time.perf_counter() - t0) / args.steps

    # Timed region: the same step captured once as a HIP graph
    # (torch.cuda.CUDAGraph) and replayed K times -- identical kernels and work
    # per step, without the per-launch host cost of the eager loop above.
    graph, graph_error = None, None
    if not args.no_graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                step()
            graph.replay()
            torch.cuda.synchronize()
        except Exception as exc:  # noqa: BLE001 - reported in the JSON line
            graph, graph_error = None, f"{type(exc).__name__}: {exc}"[:300]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    mode = "hip-graph replay" if graph is not None else "eager"

    # Per-call timing of the NF4 entry points: HIP events recorded on the
    # launch stream around every call of eager steps.  Each step is queued
    # behind a GPU spin of a few ms, so the host has enqueued the whole step
    # (events included) before the GPU reaches it and the calls run back to
    # back as in the replayed graph: the events see GPU time, not host gaps.
    timer = KernelTimer()
    cycles_per_ms = sleep_cycles_per_ms(torch)
    for name in TIMED_ENTRY_POINTS:
        _lib.hooks[name] = (timer.before, timer.after)
    for _ in range(args.timing_steps):
        torch.cuda._sleep(int(cycles_per_ms * (3 * eager_ms + 2)))
        timer.active = True
        step()
        timer.active = False
        torch.cuda.synchronize()
    _lib.hooks.clear()
    kernels = timer.summary()

    ms_per_step = 1e3 * elapsed / args.steps
    flops = layer.flops(tokens)
    for v in kernels.values():
        v["total_ms"] /= max(args.timing_steps, 1)  # per step
    value = flops / (elapsed / args.steps) / 1e12
    dominant = max(kernels, key=lambda k: kernels[k]["total_ms"])
    dk = kernels[dominant]
    traffic, source = measured_traffic().get(dominant, (None, None))
    roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(dk["tflops"], 2),
                "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(dk["tflops"] / PEAK_FP16_TFLOPS, 4), "traffic": traffic,
                "traffic_source": source,
                "avg_launch_us": round(dk["avg_us"], 3),
                "gflop_per_launch": round(dk["avg_gflop"], 4),
                "timing": (f"HIP events on the launch stream around each call, {args.timing_steps}"
                           " eager steps each queued behind a GPU spin (calls run back to back)")}

    full = None if args.no_full_layer else full_layer(torch, lengths, args.steps, args.warmup)
    sweep_res = None if args.no_sweep else sweep(torch, _lib)
    others = None if args.no_other_configs else other_configs(torch, _lib)

    cpu = None
    if not args.no_cpu_baseline:
        med, reps, threads = cpu_baseline(layer, xs, gs, args.cpu_seconds)
        cpu = {"value": round(flops / med / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
               "kind": "port", "cpu_model": cpu_model(),
               "sample": (f"{reps} full configs[1] steps (7 projections fwd+bwd, T={tokens}) of "
                          f"oracle/baseline.py: A2 decode + fp32 BLAS GEMMs; median "
                          f"{med * 1e3:.1f} ms/step")}

    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic: seeded N(0,1) fp16 activations, N(0,0.02) weights NF4-quantized "
                "on the GPU, random-init LoRA (Kaiming-uniform A, N(0,0.01) B)",
        "config": {"workload": "configs[1]: Qwen2.5-1.5B decoder layer, 7 NF4 projections + "
                               "LoRA r=16 alpha=32, fwd + dX/dA/dB bwd",
                   "tokens": tokens, "lengths": lengths, "hidden": 1536,
                   "intermediate": 8960, "kv_out": 256, "lora_rank": 16},
        "layer_fwd_bwd_ms": round(ms_per_step, 4),
        "full_decoder_layer": full,
        "step_mode": mode,
        "eager_ms_per_step": round(eager_ms, 4),
        "graph_error": graph_error,
        "nf4_weight_bytes_per_pass": layer.weight_bytes(),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in kernels.items()},
        "sweep_configs4": sweep_res,
        "other_configs": others,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
