"""Benchmark of the MI355X MatMulNBits path (one JSON line on stdout).

Workload: the Phi-3.5-mini decode layer set at M=1, int4,
block_size 32, packed uint8 zero points — qkv (K=3072, N=9216), o (3072 -> 3072), gate_up
(3072 -> 16384), down (8192 -> 3072).  One step = one token's MatMulNBits work: those four
launches over each of the model's 32 layers (128 launches, 2,098,200,576 bytes), every layer with
weights of its own, so a step streams 2.1 GB from HBM (8x the 256 MB Infinity Cache) as a real
decode does.  Inputs are synthetic (seeded), resident in HBM before the timed region.  The timed
steps are recorded once into a HIP graph and replayed, so the figure is the device's, not
Python's launch overhead (the same steps launched one by one from Python are reported as
eager_ms_per_step).

value = algorithmic bytes of one token (32 x 65,568,768 B) per step / step time, in GB/s.
The line also carries, measured in the same run:
  roofline      the dominant decode kernel's algorithmic bytes / its HIP-event launch time vs 8 TB/s
  batched_decode  the same layer set at M = 4, 8, 16 rows in GB/s of algorithmic bytes (raw
                device pointers, ORT layout), and batched_decode_session: the same through the
                session layer with the strip-major weight copy (ep.strip_major_weights)
  prefill       MatMulNBits M=2048, K=3072, N=8192 in TFLOP/s vs 2.5 PFLOP/s fp16
  accuracy_level_4  configs[4] (M=16, K=8192, N=3072, bs128, zp, int8 activations) in GB/s
  decode_f32    the layer set at M=1 with fp32 activations, scales and output in GB/s, and qkv
                on the generic kernel beside it
  prefill_f32   configs[2]'s GEMM (M = 256, 2048) with fp32 activations in TFLOP/s vs the
                157.3 TFLOP/s fp32 matrix peak
  moe           configs[3] (32 experts, top-4 of 64 tokens, gate_up and down) in GB/s
  qmoe          configs[3] as one fused QMoE op (routing, both expert GEMVs, SwiGLU, combine)
  mfma_calibration  the fp16 MFMA rate the chip sustains on random and on constant operands
  cpu_baseline  the C restatement in oracle/ (kind "port", not ORT) on the host's cores, on a
                bounded sample of the same layer set; stock_ort_cpu_baseline says whether stock
                ONNX Runtime (the reference's baseline) could be timed (it is not installed)
`--pmc-node NODE` runs one node's launches and a 256 MiB copy only, for rocprofv3 --pmc passes
(FETCH_SIZE, WRITE_SIZE) whose results give roofline.traffic (profiles/traffic_*.json).
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "onnxruntime-ep-vulkan_amd"
for _p in (str(ROOT), str(PKG)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 * 1024 * 1024
LAYERS_PER_TOKEN = 32  # Phi-3.5-mini's decoder layers: one bench step is one token

LAYER = [  # (name, K, N)
    ("qkv_proj", 3072, 9216),
    ("o_proj", 3072, 3072),
    ("gate_up_proj", 3072, 16384),
    ("down_proj", 8192, 3072),
]
BITS, BS = 4, 32


def node_bytes(m: int, k: int, n: int, bs: int = BS, zp: bool = True) -> int:
    bpc = k // bs
    b = n * k // 2 + 2 * n * bpc + (n * ((bpc * 4 + 7) // 8) if zp else 0)
    return b + 2 * m * k + 2 * m * n


def make_weights(torch, dev, k, n, gen, bs=BS, zp=True):
    """Packed int4 B [n, k/bs, bs/2], fp16 scales |N(0,1)|*0.02, packed zero points (seeded)."""
    bpc = k // bs
    B = torch.randint(0, 256, (n, bpc, bs // 2), dtype=torch.uint8, device=dev, generator=gen)
    S = (torch.randn(n * bpc, device=dev, generator=gen).abs() * 0.02).to(torch.float16)
    Z = torch.randint(0, 256, (n, (bpc * 4 + 7) // 8), dtype=torch.uint8, device=dev,
                      generator=gen) if zp else None
    return B, S, Z


def measured_traffic(node: str, algorithmic: int):
    """HBM bytes per launch of `node` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (profiles/traffic_<node>.json, each counter scaled by what it reads for a copy of known size),
    or None when no such measurement exists for this node and byte count."""
    f = ROOT / "profiles" / f"traffic_{node.removesuffix('_proj')}.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    if d.get("algorithmic_bytes_per_launch") != algorithmic:
        return None
    return d["traffic_bytes_per_launch"]


# Launch shapes over which the read floor is the least time: 1 KB runs per wavefront, wavefronts
# per workgroup, contiguous (1) or grid-stride (0) runs.
READ_SHAPES = [(l, w, c) for l in (1, 2, 4, 8, 16) for w in (4, 8, 16) for c in (1, 0)]


def graph_us(torch, stream, fn, reps: int, tries: int = 3) -> float:
    """Least average device time per call of `fn(r, stream_ptr)` over `tries` replays of one HIP
    graph of `reps` calls (HIP events on the stream the graph is replayed on)."""
    for r in range(2):
        fn(r, int(stream.cuda_stream))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(stream)
    with torch.cuda.graph(g, stream=cs):
        sp = int(torch.cuda.current_stream().cuda_stream)
        for r in range(reps):
            fn(r, sp)
    torch.cuda.synchronize()
    g.replay()
    best = float("inf")
    for _ in range(tries):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        g.replay()
        b.record(stream)
        torch.cuda.synchronize()
        best = min(best, 1e3 * a.elapsed_time(b) / reps)
    del g
    return best


def read_floor(lib, torch, dev, stream, nbytes: int, region, shapes=READ_SHAPES, reps: int = 40):
    """The least per-launch time (us) of mnb_calibrate_read over `shapes` for `nbytes`, reading a
    different copy of `region` (>= 2x the Infinity Cache) on every launch, and the best shape."""
    import mnb

    stride = -(-nbytes // 65536) * 65536
    copies = region.numel() // stride
    assert copies * nbytes >= 2 * MALL_BYTES, "region too small to rotate past the Infinity Cache"
    out = torch.zeros(1024, dtype=torch.int32, device=dev)
    best, best_shape = float("inf"), None
    for (l, w, c) in shapes:
        def f(r, sp, l=l, w=w, c=c):
            rc = lib.mnb_calibrate_read(region.data_ptr() + (r % copies) * stride, nbytes, l, w,
                                        c, out.data_ptr(), sp)
            if rc:
                mnb.check(rc)
        us = graph_us(torch, stream, f, max(reps, 2 * copies // 3))
        if us < best:
            best, best_shape = us, {"loads_per_lane": l, "waves_per_group": w,
                                    "contiguous": bool(c)}
    return best, best_shape


def cpu_baseline(seconds: float = 10.0) -> dict:
    """The oracle's C restatement on the host cores, over the same layer set at M=1."""
    import numpy as np

    so = ROOT / "oracle" / "build" / "libmnb_oracle.so"
    lib = C.CDLL(str(so))
    lib.mnb_oracle_matmul.argtypes = [C.c_void_p] * 5 + [C.c_int64] * 3 + [C.c_int] * 4
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    rng = np.random.default_rng(20260801)
    nodes = []
    for _, k, n in LAYER:
        bpc = k // BS
        nodes.append((k, n,
                      rng.standard_normal(k).astype(np.float16),
                      rng.integers(0, 256, size=n * k // 2, dtype=np.uint8),
                      (np.abs(rng.standard_normal(n * bpc)) * 0.02).astype(np.float16),
                      rng.integers(0, 256, size=n * ((bpc * 4 + 7) // 8), dtype=np.uint8),
                      np.zeros(n, dtype=np.float16)))
    per_set = sum(node_bytes(1, k, n) for _, k, n in LAYER)
    iters, t0 = 0, time.perf_counter()
    while True:
        for k, n, a, b, s, z, y in nodes:
            rc = lib.mnb_oracle_matmul(a.ctypes.data, b.ctypes.data, s.ctypes.data, z.ctypes.data,
                                       y.ctypes.data, 1, n, k, 4, BS, 1, cores)
            assert rc == 0
        iters += 1
        el = time.perf_counter() - t0
        if el >= seconds or iters >= 2000:
            break
    return {"value": round(per_set * iters / el / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"{iters} passes of the 4-node Phi-3.5 decode layer set (M=1, int4 bs32, zp) "
                      f"in {el:.1f} s with the oracle's C restatement of MatMulNBits (fp32 "
                      f"accumulate, OpenMP) -- this build's port, not ONNX Runtime"}


def stock_ort_probe() -> str:
    """Whether stock ONNX Runtime (the reference's CPU baseline) can be timed here."""
    import importlib.util

    if importlib.util.find_spec("onnxruntime") is None:
        return ("stock ORT baseline unavailable: the onnxruntime package is not installed on "
                "this machine (probed with importlib), and nothing can be installed")
    return ("onnxruntime is importable but this build does not time it: building the one-node "
            "model needs the onnx package")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--pmc-node", default=None,
                    help="counter-collection mode: launch only this decode node (qkv_proj, o_proj, "
                         "gate_up_proj, down_proj) --steps times over rotated weights, then one "
                         "plain 256 MiB device copy for calibrating FETCH_SIZE/WRITE_SIZE; no JSON")
    ap.add_argument("--pmc-launch", default=None, choices=["moe_gate_up", "moe_down", "acc4"],
                    help="counter-collection mode: launch only the MoE expert GEMV (BASELINE "
                         "configs[3], weights rotated over two copies) or the accuracy_level=4 "
                         "call (configs[4]) --steps times, then one plain 256 MiB device copy "
                         "for calibrating FETCH_SIZE/WRITE_SIZE; no JSON")
    ap.add_argument("--read-floor", action="store_true",
                    help="print, one JSON line per size, the least time one launch needs to read "
                         "that many bytes (mnb_calibrate_read over launch shapes), for the decode "
                         "nodes' byte counts and larger sizes; no benchmark line")
    ap.add_argument("--pmc-prefill", type=int, default=None, metavar="M",
                    help="counter-collection mode: launch only the prefill GEMM (K=3072, N=8192) "
                         "at M rows --steps times; no JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              f"(MatMulNBits shards along N with no collective in the hot path)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import mnb

    mnb.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=dev)
    gen.manual_seed(20260801)

    per_layer = sum(node_bytes(1, k, n) for _, k, n in LAYER)
    per_token = LAYERS_PER_TOKEN * per_layer
    copies = LAYERS_PER_TOKEN            # one weight set per layer
    layers = [[make_weights(torch, dev, k, n, gen) for _, k, n in LAYER] for _ in range(copies)]
    acts = [torch.randn(1, k, device=dev, generator=gen).to(torch.float16) for _, k, _ in LAYER]
    outs = [torch.empty(1, n, dtype=torch.float16, device=dev) for _, _, n in LAYER]
    probs = [mnb.problem(1, n, k, BITS, BS, True) for _, k, n in LAYER]
    lib = mnb.load()
    sptr = int(stream.cuda_stream)

    def launch(i, layer, sp=sptr):
        B, S, Z = layers[layer][i]
        rc = lib.mnb_matmul_nbits(C.byref(probs[i]), acts[i].data_ptr(), B.data_ptr(),
                                  S.data_ptr(), Z.data_ptr(), outs[i].data_ptr(), None, 0, sp)
        if rc:
            mnb.check(rc)

    def step(s, sp=sptr):
        for layer in range(LAYERS_PER_TOKEN):
            for i in range(len(LAYER)):
                launch(i, layer, sp)

    if args.read_floor:
        region = torch.empty(1536 << 20, dtype=torch.uint8, device=dev)
        region.random_(generator=gen)
        sizes = [(name, node_bytes(1, k, n)) for name, k, n in LAYER]
        sizes += [("acc4", node_bytes(16, 8192, 3072, bs=128))]
        sizes += [(f"{mb} MiB", mb << 20) for mb in (1, 2, 4, 8, 32, 64, 128, 256, 512)]
        for name, nb in sizes:
            us, shape = read_floor(lib, torch, dev, stream, nb, region)
            print(json.dumps({"size": name, "bytes": nb, "floor_us": round(us, 3),
                              "GB/s": round(nb / (us * 1e-6) / 1e9, 1),
                              "frac_of_peak": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                              "shape": shape}), flush=True)
        return 0

    if args.pmc_prefill:
        pm, pk, pn = args.pmc_prefill, 3072, 8192
        pw = [make_weights(torch, dev, pk, pn, gen, zp=False) for _ in range(2)]
        pA = torch.randn(pm, pk, device=dev, generator=gen).to(torch.float16)
        pY = torch.empty(pm, pn, dtype=torch.float16, device=dev)
        pprob = mnb.problem(pm, pn, pk, BITS, BS, False)
        pwsb = mnb.workspace_bytes(pprob)
        pws = torch.empty(max(pwsb, 1), dtype=torch.uint8, device=dev)
        for r in range(args.steps):
            pB, pS, _ = pw[r % 2]
            mnb.check(lib.mnb_matmul_nbits(C.byref(pprob), pA.data_ptr(), pB.data_ptr(),
                                           pS.data_ptr(), None, pY.data_ptr(), pws.data_ptr(),
                                           pwsb, sptr))
        torch.cuda.synchronize()
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"pmc mode: {args.steps} launches of the prefill GEMM M={pm} K={pk} N={pn} "
              f"({mnb.KERNEL_NAMES.get(mnb.plan(pprob).kernel)}), then one copy of "
              f"{src.numel()} bytes")
        return 0

    if args.pmc_launch:
        if args.pmc_launch == "acc4":
            ak, an, am, abs_ = 8192, 3072, 16, 128
            a_copies = max(2, -(-2 * MALL_BYTES // node_bytes(am, ak, an, bs=abs_)))
            a_w = [make_weights(torch, dev, ak, an, gen, bs=abs_) for _ in range(a_copies)]
            a_A = torch.randn(am, ak, device=dev, generator=gen).to(torch.float16)
            a_Y = torch.empty(am, an, dtype=torch.float16, device=dev)
            a_prob = mnb.problem(am, an, ak, BITS, abs_, True, mnb.DTYPE_F16, 4)
            a_ws = torch.empty(mnb.workspace_bytes(a_prob), dtype=torch.uint8, device=dev)
            for r in range(args.steps):
                B, S, Z = a_w[r % a_copies]
                mnb.check(lib.mnb_matmul_nbits(C.byref(a_prob), a_A.data_ptr(), B.data_ptr(),
                                               S.data_ptr(), Z.data_ptr(), a_Y.data_ptr(),
                                               a_ws.data_ptr(), a_ws.numel(), sptr))
            what = f"accuracy_level=4 M={am} K={ak} N={an} bs{abs_} ({node_bytes(am, ak, an, bs=abs_)} algorithmic bytes)"
        else:
            E, T, TOPK, MK = 32, 64, 4, 2880
            mn = 5760 if args.pmc_launch == "moe_gate_up" else 2880
            top = np.argsort(-np.random.default_rng(20260801).standard_normal((T, E)), axis=1,
                             kind="stable")[:, :TOPK].reshape(-1)
            rows = torch.from_numpy((np.argsort(top, kind="stable") // TOPK).astype(np.int32)).to(dev)
            cnt = np.bincount(top, minlength=E)
            off = torch.from_numpy(np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)).to(dev)
            mA = torch.randn(T, MK, device=dev, generator=gen).to(torch.float16)
            bpc = MK // BS
            wB = [torch.randint(0, 256, (E, mn, bpc, BS // 2), dtype=torch.uint8, device=dev,
                                generator=gen) for _ in range(2)]
            wS = [(torch.randn(E, mn * bpc, device=dev, generator=gen).abs() * 0.02).to(torch.float16)
                  for _ in range(2)]
            mY = torch.empty(T * TOPK, mn, dtype=torch.float16, device=dev)
            mp = mnb.MoeProblem(E, T * TOPK, int(cnt.max()), T, mn, MK, BITS, BS, 0, mnb.DTYPE_F16)
            for r in range(args.steps):
                mnb.check(lib.mnb_moe_grouped(C.byref(mp), mA.data_ptr(), rows.data_ptr(),
                                              off.data_ptr(), wB[r % 2].data_ptr(),
                                              wS[r % 2].data_ptr(), None, mY.data_ptr(), sptr))
            what = f"MoE {args.pmc_launch} ({E * (mn * MK // 2 + 2 * mn * bpc)} bytes of expert weights and scales)"
        torch.cuda.synchronize()
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"pmc mode: {args.steps} launches of {what}, then one copy of {src.numel()} bytes")
        return 0

    if args.pmc_node:
        i = [x[0] for x in LAYER].index(args.pmc_node)
        for s in range(args.steps):
            launch(i, s % copies)
        torch.cuda.synchronize()
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"pmc mode: {args.steps} launches of {args.pmc_node} "
              f"({node_bytes(1, LAYER[i][1], LAYER[i][2])} algorithmic bytes each), "
              f"then one copy of {src.numel()} bytes")
        return 0

    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()
    eager_out = [o.clone() for o in outs]          # outputs of step warmup-1

    # The step's launches are recorded once into a HIP graph (stream capture on a side stream)
    # so that the timed region measures the device, not Python's per-launch overhead.
    def capture(fn):
        g = torch.cuda.CUDAGraph()
        cs = torch.cuda.Stream()
        cs.wait_stream(stream)
        with torch.cuda.graph(g, stream=cs):
            fn(int(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        return g

    graph = capture(lambda sp: [step(s, sp) for s in range(args.steps)])
    graph.replay()
    torch.cuda.synchronize()
    # every step launches the same 128 nodes: one eager step must reproduce the graph's outputs
    for s in range(args.steps - 1, args.steps):
        step(s)
    torch.cuda.synchronize()
    ref_out = [o.clone() for o in outs]
    graph.replay()
    torch.cuda.synchronize()
    for o, r in zip(outs, ref_out):
        if not torch.equal(o, r):
            raise RuntimeError("graph replay and eager launches disagree")
    del eager_out

    # Timed region: exactly `steps` steps of the four launches (one graph replay), bracketed by
    # a synchronize on both sides (wall clock) and by two HIP events on the stream (device time).
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    graph.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    dev_ms_step = ev0.elapsed_time(ev1) / args.steps
    value = per_token / (ms_step * 1e-3) / 1e9

    # The same steps launched one by one from Python (reported, not the value).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(s)
    torch.cuda.synchronize()
    eager_ms_step = (time.perf_counter() - t0) * 1e3 / args.steps

    # Per-node launch duration: HIP events around a graph of `reps` back-to-back launches of one
    # node (weights rotated as in the step: "cold", from HBM), divided by `reps`: each launch's
    # device time including the gap to the next launch on the stream.
    reps = max(20, copies * 4)
    kern_us = []
    for i in range(len(LAYER)):
        g1 = capture(lambda sp, i=i: [launch(i, r % copies, sp) for r in range(reps)])
        g1.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        g1.replay()
        b.record(stream)
        torch.cuda.synchronize()
        kern_us.append(1e3 * a.elapsed_time(b) / reps)
        del g1
    # The same launches on one weight copy every time ("hot": the 5-29 MB of weights stay in
    # the 256 MB Infinity Cache), reported beside the rotated ("cold", HBM) times.
    hot_us = []
    for i in range(len(LAYER)):
        g1 = capture(lambda sp, i=i: [launch(i, 0, sp) for _ in range(reps)])
        g1.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        g1.replay()
        b.record(stream)
        torch.cuda.synchronize()
        hot_us.append(1e3 * a.elapsed_time(b) / reps)
        del g1

    # The read floor of each node's byte count: the least time one launch of a kernel that does
    # nothing but read that many bytes (all loads issued up front) needs on this device, over
    # launch shapes, reading a fresh copy on every launch as the decode launches do.
    region = torch.empty(768 << 20, dtype=torch.uint8, device=dev)
    region.random_(generator=gen)
    floors = [read_floor(lib, torch, dev, stream, node_bytes(1, k, n), region)
              for _, k, n in LAYER]
    del region

    per_kernel = []
    for i, ((name, k, n), us) in enumerate(zip(LAYER, kern_us)):
        nb = node_bytes(1, k, n)
        per_kernel.append({"node": name, "K": k, "N": n, "bytes": nb, "us": round(us, 3),
                           "GB/s": round(nb / (us * 1e-6) / 1e9, 1),
                           "frac_hbm": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                           "hot_us": round(hot_us[i], 3),
                           "read_floor_us": round(floors[i][0], 3),
                           "frac_of_read_floor": round(floors[i][0] / us, 4),
                           "kernel": mnb.KERNEL_NAMES.get(mnb.plan(probs[i]).kernel, "?")})
    # the token's time as the sum of its launches, each timed on its own (32 x the four nodes)
    node_sum_ms = LAYERS_PER_TOKEN * sum(kern_us) * 1e-3
    dom = max(range(len(LAYER)), key=lambda i: kern_us[i])
    dom_bytes = node_bytes(1, LAYER[dom][1], LAYER[dom][2])
    achieved = dom_bytes / (kern_us[dom] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(LAYER[dom][0], dom_bytes),
                "kernel": f"MatMulNBits {LAYER[dom][0]} M=1 K={LAYER[dom][1]} N={LAYER[dom][2]}",
                "per_launch_bytes": dom_bytes, "launch_us": round(kern_us[dom], 3),
                "read_floor_us": round(floors[dom][0], 3),
                "read_floor_shape": floors[dom][1],
                "frac_of_read_floor": round(floors[dom][0] / kern_us[dom], 4)}

    # Batched decode: the same layer set at 4, 8 and 16 rows (the north star's M = 1..16 decode
    # range; not part of `value`).  Per node, HIP events around a graph of `reps` launches with
    # the weights rotated as in the step; the layer time is the sum over the four nodes.
    bacts = [torch.randn(16, k, device=dev, generator=gen).to(torch.float16) for _, k, _ in LAYER]
    bouts = [torch.empty(16, n, dtype=torch.float16, device=dev) for _, _, n in LAYER]
    batched = []
    for bm in (4, 8, 16):
        bprobs = [mnb.problem(bm, n, k, BITS, BS, True) for _, k, n in LAYER]

        def blaunch(i, layer, sp, bprobs=bprobs):
            B, S, Z = layers[layer][i]
            rc = lib.mnb_matmul_nbits(C.byref(bprobs[i]), bacts[i].data_ptr(), B.data_ptr(),
                                      S.data_ptr(), Z.data_ptr(), bouts[i].data_ptr(), None, 0, sp)
            if rc:
                mnb.check(rc)
        node_us = []
        for i in range(len(LAYER)):
            g1 = capture(lambda sp, i=i: [blaunch(i, r % copies, sp) for r in range(reps)])
            g1.replay()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record(stream)
            g1.replay()
            b.record(stream)
            torch.cuda.synchronize()
            node_us.append(1e3 * a.elapsed_time(b) / reps)
            del g1
        bbytes = sum(node_bytes(bm, k, n) for _, k, n in LAYER)
        batched.append({"M": bm, "layer_us": round(sum(node_us), 3),
                        "GB/s": round(bbytes / (sum(node_us) * 1e-6) / 1e9, 1),
                        "frac_hbm": round(bbytes / (sum(node_us) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        "node_us": {LAYER[i][0]: round(u, 3) for i, u in enumerate(node_us)},
                        "kernels": sorted({mnb.KERNEL_NAMES.get(mnb.plan(bp).kernel, "?")
                                           for bp in bprobs})})

    # The same batched decode through the session layer, as the EP runs it with
    # the EP's default (ep.strip_major_weights): each node's weights uploaded once (mnb_weights_upload) with their
    # strip-major copy (mnb_weights_prepack), then mnb_session_run_device on the session's own
    # stream; a graph of launches per node on that stream, weights rotated over the same 32
    # layer copies as the raw launches above.
    sess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(sess)))
    sstream = torch.cuda.ExternalStream(int(lib.mnb_session_stream(sess)))
    scopies = copies
    sw = []
    for c in range(scopies):
        row = []
        for i, (_, k, n) in enumerate(LAYER):
            B, S, Z = (t.cpu().numpy() for t in layers[c][i])
            w = C.c_void_p()
            p0 = mnb.problem(0, n, k, BITS, BS, True)
            mnb.check(lib.mnb_weights_upload(sess, C.byref(p0), B.ctypes.data, B.nbytes,
                                             S.ctypes.data, S.nbytes, Z.ctypes.data, Z.nbytes,
                                             C.byref(w)))
            mnb.check(lib.mnb_weights_prepack(w, None))
            row.append(w)
        sw.append(row)
    batched_session = []
    for bm in (4, 8, 16):
        node_us = []
        for i in range(len(LAYER)):
            def slaunch(r, i=i, bm=bm):
                rc = lib.mnb_session_run_device(sess, sw[r % scopies][i], bm, bacts[i].data_ptr(),
                                                bouts[i].data_ptr())
                if rc:
                    mnb.check(rc)
            for r in range(2):
                slaunch(r)
            torch.cuda.synchronize()
            g1 = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g1, stream=sstream):
                for r in range(reps):
                    slaunch(r)
            # a replay runs on the stream current at the call (here `stream`): time it there
            g1.replay()
            best = float("inf")
            for _ in range(3):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                a.record(stream)
                g1.replay()
                b.record(stream)
                torch.cuda.synchronize()
                best = min(best, 1e3 * a.elapsed_time(b) / reps)
            node_us.append(best)
            del g1
        bbytes = sum(node_bytes(bm, k, n) for _, k, n in LAYER)
        batched_session.append({
            "M": bm, "layer_us": round(sum(node_us), 3),
            "GB/s": round(bbytes / (sum(node_us) * 1e-6) / 1e9, 1),
            "frac_hbm": round(bbytes / (sum(node_us) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "node_us": {LAYER[i][0]: round(u, 3) for i, u in enumerate(node_us)}})
    for row in sw:
        for w in row:
            lib.mnb_weights_release(w)
    lib.mnb_session_destroy(sess)
    del bacts, bouts

    # Prefill: M in {256, 512, 2048}, K=3072, N=8192, implicit zero point
    # (not part of `value`).  HIP events around a graph of `preps` launches; weights rotate over
    # two copies so consecutive launches do not reuse an L2-resident B.
    pk, pn = 3072, 8192
    pw = [make_weights(torch, dev, pk, pn, gen, zp=False) for _ in range(2)]

    # The fp16 MFMA rate the chip sustains on its own (mnb_calibrate_mfma: 16 independent
    # accumulators per wavefront, no memory traffic), once on random N(0,1) operands and once on
    # constant ones.  Under a full-chip MFMA load the clock follows the power the matrix cores
    # draw, so random data (the prefill GEMM's kind) runs well below the nominal peak.
    def mfma_ceiling(random_operands: bool, wgs: int = 512, iters: int = 1000) -> float:
        ops = (torch.randn(wgs * 256 * 64, device=dev, generator=gen).to(torch.float16)
               if random_operands else None)
        out = torch.empty(wgs * 256, dtype=torch.float32, device=dev)

        def call():
            mnb.check(lib.mnb_calibrate_mfma(wgs, iters, None if ops is None else ops.data_ptr(),
                                             out.data_ptr(), sptr))
        call()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(3):
            call()
        b.record(stream)
        torch.cuda.synchronize()
        us = 1e3 * a.elapsed_time(b) / 3
        return wgs * 4 * iters * 16 * 32768 / (us * 1e-6) / 1e12

    ceil_rand = mfma_ceiling(True)
    ceil_const = mfma_ceiling(False)
    # the same loop on 32 workgroups (32 of the 256 CUs), scaled to the whole chip: the per-CU
    # rate when the chip is far from its power limit
    ceil_rand32 = mfma_ceiling(True, wgs=32) * 256 / 32
    mfma_cal = {"random_operands_tflops": round(ceil_rand, 1),
                "constant_operands_tflops": round(ceil_const, 1),
                "random_operands_32_cus_scaled_tflops": round(ceil_rand32, 1),
                "nominal_peak_tflops": F16_MFMA_PEAK_TFLOPS,
                "kernel": "mnb_calibrate_mfma: 512 workgroups x 4 wavefronts x 1000 x 16 "
                          "v_mfma_f32_32x32x16_f16, operands in registers"}
    prefill = []
    for pm in (256, 512, 2048):
        pA = torch.randn(pm, pk, device=dev, generator=gen).to(torch.float16)
        pY = torch.empty(pm, pn, dtype=torch.float16, device=dev)
        pprob = mnb.problem(pm, pn, pk, BITS, BS, False)
        pinfo = mnb.plan(pprob)
        # the K-split partials of the GEMM at M < 1024 (fewer row tiles than CUs)
        pwsb = mnb.workspace_bytes(pprob)
        pws = torch.empty(max(pwsb, 1), dtype=torch.uint8, device=dev)

        def plaunch(r, sp, pA=pA, pY=pY, pprob=pprob, pws=pws, pwsb=pwsb):
            pB, pS, _ = pw[r % 2]
            rc = lib.mnb_matmul_nbits(C.byref(pprob), pA.data_ptr(), pB.data_ptr(),
                                      pS.data_ptr(), None, pY.data_ptr(), pws.data_ptr(), pwsb,
                                      sp)
            if rc:
                mnb.check(rc)

        preps = 20
        for r in range(3):
            plaunch(r, sptr)
        pg = capture(lambda sp: [plaunch(r, sp) for r in range(preps)])
        pg.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        pg.replay()
        b.record(stream)
        torch.cuda.synchronize()
        pus = 1e3 * a.elapsed_time(b) / preps
        del pg
        ptf = 2.0 * pm * pn * pk / (pus * 1e-6) / 1e12
        prefill.append({"M": pm, "K": pk, "N": pn, "us": round(pus, 2), "TFLOP/s": round(ptf, 2),
                        "kernel": mnb.KERNEL_NAMES.get(pinfo.kernel, "?"),
                        "tile": [pinfo.tile_m, pinfo.tile_n],
                        "k_split": pinfo.grid_x // ((pm + pinfo.tile_m - 1) // pinfo.tile_m
                                                    * ((pn + pinfo.tile_n - 1) // pinfo.tile_n)),
                        "roofline": {"bound": "mfma", "achieved": round(ptf, 2),
                                     "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                     "frac": round(ptf / F16_MFMA_PEAK_TFLOPS, 4),
                                     "traffic": measured_traffic(
                                         f"prefill_m{pm}",
                                         pm * pk * 2 + pn * pk // 2 + pn * (pk // BS) * 2
                                         + pm * pn * 2),
                                     "ceiling_random_operands": round(ceil_rand, 1),
                                     "frac_of_ceiling": round(ptf / ceil_rand, 4)}})

    # 8-bit prefill: gpt-oss's 8-bit MatMulNBits nodes (bits 8, block 32, zero points) at the
    # prefill GEMM's M=2048, K = N = 2880; weights rotate over two copies.
    qk8, qn8, qm8, qbs8 = 2880, 2880, 2048, 32
    bpc8 = qk8 // qbs8
    w8 = [(torch.randint(0, 256, (qn8, bpc8, qbs8), dtype=torch.uint8, device=dev, generator=gen),
           (torch.randn(qn8 * bpc8, device=dev, generator=gen).abs() * 0.02).to(torch.float16),
           torch.randint(0, 256, (qn8, bpc8), dtype=torch.uint8, device=dev, generator=gen))
          for _ in range(2)]
    A8 = torch.randn(qm8, qk8, device=dev, generator=gen).to(torch.float16)
    Y8 = torch.empty(qm8, qn8, dtype=torch.float16, device=dev)
    p8 = mnb.problem(qm8, qn8, qk8, 8, qbs8, True)
    ws8b = mnb.workspace_bytes(p8)
    ws8 = torch.empty(max(ws8b, 1), dtype=torch.uint8, device=dev)

    def launch8(r, sp):
        B8, S8, Z8 = w8[r % 2]
        rc = lib.mnb_matmul_nbits(C.byref(p8), A8.data_ptr(), B8.data_ptr(), S8.data_ptr(),
                                  Z8.data_ptr(), Y8.data_ptr(), ws8.data_ptr(), ws8b, sp)
        if rc:
            mnb.check(rc)

    us8 = graph_us(torch, stream, launch8, 20)
    tf8 = 2.0 * qm8 * qn8 * qk8 / (us8 * 1e-6) / 1e12
    prefill_8bit = {"M": qm8, "K": qk8, "N": qn8, "bits": 8, "block_size": qbs8,
                    "zero_points": True, "us": round(us8, 2), "TFLOP/s": round(tf8, 2),
                    "kernel": mnb.KERNEL_NAMES.get(mnb.plan(p8).kernel, "?"),
                    "roofline": {"bound": "mfma", "achieved": round(tf8, 2),
                                 "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(tf8 / F16_MFMA_PEAK_TFLOPS, 4),
                                 "traffic": None,
                                 "ceiling_random_operands": round(ceil_rand, 1),
                                 "frac_of_ceiling": round(tf8 / ceil_rand, 4)}}
    del w8

    def graph_time_us(fn, reps):
        """Average device time per launch of `fn(r, stream)` over a graph of `reps` launches."""
        for r in range(2):
            fn(r, sptr)
        g = capture(lambda sp: [fn(r, sp) for r in range(reps)])
        g.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        g.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return 1e3 * a.elapsed_time(b) / reps

    # accuracy_level = 4: M=16, K=8192, N=3072, int4 bs128 with zero points;
    # one call = the int8 quantiser of A + the int8 MFMA GEMV.  Weights rotated over >= 2x MALL.
    ak, an, am, abs_ = 8192, 3072, 16, 128
    a_bytes = node_bytes(am, ak, an, bs=abs_)
    a_copies = max(2, -(-2 * MALL_BYTES // a_bytes))
    a_w = [make_weights(torch, dev, ak, an, gen, bs=abs_) for _ in range(a_copies)]
    a_A = torch.randn(am, ak, device=dev, generator=gen).to(torch.float16)
    a_Y = torch.empty(am, an, dtype=torch.float16, device=dev)
    a_prob = mnb.problem(am, an, ak, BITS, abs_, True, mnb.DTYPE_F16, 4)
    a_ws_bytes = mnb.workspace_bytes(a_prob)
    a_ws = torch.empty(a_ws_bytes, dtype=torch.uint8, device=dev)

    def alaunch(r, sp):
        B, S, Z = a_w[r % a_copies]
        rc = lib.mnb_matmul_nbits(C.byref(a_prob), a_A.data_ptr(), B.data_ptr(), S.data_ptr(),
                                  Z.data_ptr(), a_Y.data_ptr(), a_ws.data_ptr(), a_ws_bytes, sp)
        if rc:
            mnb.check(rc)

    a_us = graph_time_us(alaunch, max(20, 2 * a_copies))
    acc4 = {"config": "M=16 K=8192 N=3072 int4 bs128 zp, accuracy_level=4", "bytes": a_bytes,
            "us": round(a_us, 3), "GB/s": round(a_bytes / (a_us * 1e-6) / 1e9, 1),
            "int_TOPS": round(2.0 * am * an * ak / (a_us * 1e-6) / 1e12, 2),
            "kernel": "quantize_a_int8 + " + {
                mnb.KERNEL_ACC4_STREAM: "acc4_stream (one 16-column strip per workgroup over "
                                        "all of K, int8 MFMA)",
            }.get(mnb.plan(a_prob).kernel, mnb.KERNEL_NAMES.get(mnb.plan(a_prob).kernel, "?")),
            "roofline": {"bound": "hbm", "achieved": round(a_bytes / (a_us * 1e-6) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(a_bytes / (a_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}}

    # The same calls through the session layer with each copy's strip-major weights
    # (mnb_weights_prepack, as the EP keeps them by default).
    asess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(asess)))
    astream = torch.cuda.ExternalStream(int(lib.mnb_session_stream(asess)))
    aw = []
    for (B, S, Z) in a_w:
        Bh, Sh, Zh = B.cpu().numpy(), S.cpu().numpy(), Z.cpu().numpy()
        p0 = mnb.problem(0, an, ak, BITS, abs_, True, mnb.DTYPE_F16, 4)
        w = C.c_void_p()
        mnb.check(lib.mnb_weights_upload(asess, C.byref(p0), Bh.ctypes.data, Bh.nbytes,
                                         Sh.ctypes.data, Sh.nbytes, Zh.ctypes.data, Zh.nbytes,
                                         C.byref(w)))
        mnb.check(lib.mnb_weights_prepack(w, None))
        aw.append(w)

    def aslaunch(r):
        rc = lib.mnb_session_run_device(asess, aw[r % a_copies], am, a_A.data_ptr(),
                                        a_Y.data_ptr())
        if rc:
            mnb.check(rc)
    areps = max(20, 2 * a_copies)
    for r in range(2):
        aslaunch(r)
    torch.cuda.synchronize()
    ag = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ag, stream=astream):
        for r in range(areps):
            aslaunch(r)
    ag.replay()
    as_us = float("inf")
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        ag.replay()                      # a replay runs on the current stream: timed there
        b.record(stream)
        torch.cuda.synchronize()
        as_us = min(as_us, 1e3 * a.elapsed_time(b) / areps)
    del ag
    for w in aw:
        lib.mnb_weights_release(w)
    lib.mnb_session_destroy(asess)
    acc4["session_strip_major"] = {
        "path": "mnb_weights_upload + mnb_weights_prepack, mnb_session_run_device",
        "us": round(as_us, 3), "GB/s": round(a_bytes / (as_us * 1e-6) / 1e9, 1),
        "frac_hbm": round(a_bytes / (as_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del a_w

    # fp32 activations, scales and output (the form of ORT's CPU-exported int4 models): the
    # Phi-3.5 layer set at M=1 through mnb_matmul_nbits, the same packed weights and zero points
    # with fp32 scales, rotated over the 32 layer copies; qkv also on the generic kernel, which
    # every fp32 call ran before the fp32 streaming GEMV.
    f_scales = [[S.float() for (_, S, _) in layer] for layer in layers]
    f_acts = [torch.randn(1, k, device=dev, generator=gen) for _, k, _ in LAYER]
    f_outs = [torch.empty(1, n, dtype=torch.float32, device=dev) for _, _, n in LAYER]
    f_probs = [mnb.problem(1, n, k, BITS, BS, True, mnb.DTYPE_F32) for _, k, n in LAYER]

    def f32_bytes(k, n):
        bpc = k // BS
        return n * k // 2 + 4 * n * bpc + n * ((bpc * 4 + 7) // 8) + 4 * k + 4 * n

    def flaunch(i, r, sp):
        B, _, Z = layers[r % copies][i]
        rc = lib.mnb_matmul_nbits(C.byref(f_probs[i]), f_acts[i].data_ptr(), B.data_ptr(),
                                  f_scales[r % copies][i].data_ptr(), Z.data_ptr(),
                                  f_outs[i].data_ptr(), None, 0, sp)
        if rc:
            mnb.check(rc)

    f32_nodes = []
    for i, (name, k, n) in enumerate(LAYER):
        us = graph_time_us(lambda r, sp, i=i: flaunch(i, r, sp), reps)
        nb = f32_bytes(k, n)
        f32_nodes.append({"node": name, "bytes": nb, "us": round(us, 3),
                          "GB/s": round(nb / (us * 1e-6) / 1e9, 1),
                          "frac_hbm": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "kernel": mnb.KERNEL_NAMES.get(mnb.plan(f_probs[i]).kernel, "?")})
    f_layer_us = sum(x["us"] for x in f32_nodes)
    f_layer_bytes = sum(x["bytes"] for x in f32_nodes)
    old_force = os.environ.get("MNB_FORCE_KERNEL")
    os.environ["MNB_FORCE_KERNEL"] = "generic"
    try:
        f_generic_us = graph_time_us(lambda r, sp: flaunch(0, r, sp), 8)
    finally:
        if old_force is None:
            os.environ.pop("MNB_FORCE_KERNEL", None)
        else:
            os.environ["MNB_FORCE_KERNEL"] = old_force
    decode_f32 = {"config": "Phi-3.5 decode layer set, M=1, fp32 A / scales / Y, int4 bs32 zp",
                  "nodes": f32_nodes, "layer_us": round(f_layer_us, 3),
                  "GB/s": round(f_layer_bytes / (f_layer_us * 1e-6) / 1e9, 1),
                  "frac_hbm": round(f_layer_bytes / (f_layer_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                  "qkv_generic_us": round(f_generic_us, 3)}
    del f_scales

    # fp32 prefill: configs[2]'s GEMM shape with fp32 activations, scales and output, on the
    # fp32 MFMA GEMM (weights dequantised exactly to fp32 in LDS), against the fp32 matrix peak.
    F32_MFMA_PEAK_TFLOPS = 157.3
    prefill_f32 = []
    for pm in (256, 2048):
        pk, pn = 3072, 8192
        pw = [make_weights(torch, dev, pk, pn, gen, zp=False) for _ in range(2)]
        pS = [S.float() for (_, S, _) in pw]
        pA = torch.randn(pm, pk, device=dev, generator=gen)
        pY = torch.empty(pm, pn, dtype=torch.float32, device=dev)
        pprob = mnb.problem(pm, pn, pk, BITS, BS, False, mnb.DTYPE_F32)

        def plaunch(r, sp):
            rc = lib.mnb_matmul_nbits(C.byref(pprob), pA.data_ptr(), pw[r % 2][0].data_ptr(),
                                      pS[r % 2].data_ptr(), None, pY.data_ptr(), None, 0, sp)
            if rc:
                mnb.check(rc)

        us = graph_time_us(plaunch, 10)
        tf = 2.0 * pm * pn * pk / (us * 1e-6) / 1e12
        prefill_f32.append({"M": pm, "K": pk, "N": pn, "us": round(us, 2), "TFLOP/s": round(tf, 1),
                            "kernel": mnb.KERNEL_NAMES.get(mnb.plan(pprob).kernel, "?") + " (fp32)",
                            "roofline": {"bound": "mfma", "achieved": round(tf, 1),
                                         "peak": F32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                         "frac": round(tf / F32_MFMA_PEAK_TFLOPS, 4)}})
        del pw, pS, pA, pY

    # gpt-oss-shaped MoE: 32 experts, 64 tokens, softmax top-4 routing of
    # N(0,1) logits (seeded), per-expert int4 bs32 gate_up (2880 -> 5760) and down (2880 -> 2880).
    E, T, TOPK, MK = 32, 64, 4, 2880
    rng = np.random.default_rng(20260801)
    logits = rng.standard_normal((T, E))
    top = np.argsort(-logits, axis=1, kind="stable")[:, :TOPK]        # softmax is monotone
    flat = top.reshape(-1)
    order = np.argsort(flat, kind="stable")
    m_rows = torch.from_numpy((order // TOPK).astype(np.int32)).to(dev)
    counts = np.bincount(flat, minlength=E)
    m_off = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).to(dev)
    m_A = torch.randn(T, MK, device=dev, generator=gen).to(torch.float16)
    moe = []
    for name, mn in (("gate_up", 5760), ("down", 2880)):
        bpc = MK // BS
        wB = [torch.randint(0, 256, (E, mn, bpc, BS // 2), dtype=torch.uint8, device=dev,
                            generator=gen) for _ in range(2)]
        wS = [(torch.randn(E, mn * bpc, device=dev, generator=gen).abs() * 0.02).to(torch.float16)
              for _ in range(2)]
        mY = torch.empty(T * TOPK, mn, dtype=torch.float16, device=dev)
        mp = mnb.MoeProblem(E, T * TOPK, int(counts.max()), T, mn, MK, BITS, BS, 0, mnb.DTYPE_F16)
        wbytes = E * (mn * MK // 2 + 2 * mn * bpc)
        mbytes = wbytes + 2 * T * MK + 2 * T * TOPK * mn

        def mlaunch(r, sp, wB=wB, wS=wS, mY=mY, mp=mp):
            rc = lib.mnb_moe_grouped(C.byref(mp), m_A.data_ptr(), m_rows.data_ptr(),
                                     m_off.data_ptr(), wB[r % 2].data_ptr(), wS[r % 2].data_ptr(),
                                     None, mY.data_ptr(), sp)
            if rc:
                mnb.check(rc)

        m_us = graph_time_us(mlaunch, 10)
        moe.append({"node": name, "K": MK, "N": mn, "experts": E, "bytes": mbytes,
                    "us": round(m_us, 2), "GB/s": round(mbytes / (m_us * 1e-6) / 1e9, 1),
                    "frac_hbm": round(mbytes / (m_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del wB, wS

    # The whole gpt-oss QMoE layer of configs[3] as one fused op (mnb_qmoe): device routing of
    # the same 64 x 32 N(0,1) logits, fc1 (gate_up, with bias) + SwiGLU (alpha 1.702, beta 1,
    # limit 7, interleaved) + fc2 (down, with bias) + weighted combine.  Expert tensors rotated
    # over two copies (896 MB > 2x MALL).  Algorithmic bytes: all 32 experts' weights, scales
    # and biases (every expert is routed to with near certainty), x, the logits and y.
    q_I = 2880
    q_prob = mnb.qmoe_problem(T, MK, q_I, E, TOPK, BS, 1, True, 1.702, 1.0, 7.0)
    q_ws_n = C.c_size_t(0)
    mnb.check(lib.mnb_qmoe_workspace_bytes(C.byref(q_prob), C.byref(q_ws_n)))
    q_ws = torch.empty(int(q_ws_n.value), dtype=torch.uint8, device=dev)
    q_x = torch.randn(T, MK, device=dev, generator=gen).to(torch.float16)
    q_lg = torch.from_numpy(logits.astype(np.float16)).to(dev)
    q_y = torch.empty(T, MK, dtype=torch.float16, device=dev)

    def qtensors():
        w1 = torch.randint(0, 256, (E, 2 * q_I, MK // 2), dtype=torch.uint8, device=dev, generator=gen)
        s1 = (torch.randn(E, 2 * q_I, MK // BS, device=dev, generator=gen).abs() * 0.02).to(torch.float16)
        b1 = (torch.randn(E, 2 * q_I, device=dev, generator=gen) * 0.1).to(torch.float16)
        w2 = torch.randint(0, 256, (E, MK, q_I // 2), dtype=torch.uint8, device=dev, generator=gen)
        s2 = (torch.randn(E, MK, q_I // BS, device=dev, generator=gen).abs() * 0.02).to(torch.float16)
        b2 = (torch.randn(E, MK, device=dev, generator=gen) * 0.1).to(torch.float16)
        return w1, s1, b1, w2, s2, b2

    q_w = [qtensors() for _ in range(2)]
    q_bytes = sum(t.numel() * t.element_size() for t in q_w[0]) + 2 * T * MK * 2 + 2 * T * E

    def qlaunch(r, sp):
        w1, s1, b1, w2, s2, b2 = q_w[r % 2]
        rc = lib.mnb_qmoe(C.byref(q_prob), q_x.data_ptr(), q_lg.data_ptr(), w1.data_ptr(),
                          s1.data_ptr(), b1.data_ptr(), w2.data_ptr(), s2.data_ptr(),
                          b2.data_ptr(), q_y.data_ptr(), q_ws.data_ptr(), q_ws.numel(), sp)
        if rc:
            mnb.check(rc)

    q_us = graph_time_us(qlaunch, 10)
    qmoe = {"config": "gpt-oss-20b QMoE layer: 64 tokens, 32 experts, top-4, H = I = 2880, "
                      "int4 bs32, biases, SwiGLU alpha 1.702 beta 1 limit 7",
            "bytes": q_bytes, "us": round(q_us, 2),
            "GB/s": round(q_bytes / (q_us * 1e-6) / 1e9, 1),
            "kernels": "qmoe_topk + strip_gemv (fc1: finds its expert's rows from the "
                       "routing, SwiGLU applied as its tiles are stored) + strip_gemv (fc2) + "
                       "qmoe_combine",
            "roofline": {"bound": "hbm", "achieved": round(q_bytes / (q_us * 1e-6) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(q_bytes / (q_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}}

    # The same layer through the session layer as the EP runs it by default (ep.strip_major_weights):
    # both weight copies uploaded (mnb_qmoe_weights_upload) with their strip-major expert
    # weights (mnb_qmoe_weights_prepack); an async session, so device-resident calls return
    # once enqueued and can be recorded into a graph on the session's stream.
    qsess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(qsess)))
    mnb.check(lib.mnb_session_set_async(qsess, 1))
    qstream = torch.cuda.ExternalStream(int(lib.mnb_session_stream(qsess)))
    qsw = []
    for tens in q_w:
        host = [t.cpu().numpy() for t in tens]
        w = C.c_void_p()
        p0 = mnb.qmoe_problem(0, MK, q_I, E, TOPK, BS, 1, True, 1.702, 1.0, 7.0)
        mnb.check(lib.mnb_qmoe_weights_upload(qsess, C.byref(p0), 0,
                                              *[v for h in host for v in (h.ctypes.data, h.nbytes)],
                                              C.byref(w)))
        mnb.check(lib.mnb_qmoe_weights_prepack(w, None))
        qsw.append(w)
        del host

    def qslaunch(r):
        rc = lib.mnb_session_run_qmoe(qsess, qsw[r % 2], T, q_x.data_ptr(), 1, q_lg.data_ptr(), 1,
                                      q_y.data_ptr(), 1)
        if rc:
            mnb.check(rc)
    for r in range(2):
        qslaunch(r)
    torch.cuda.synchronize()
    lib.mnb_session_synchronize(qsess)
    qg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(qg, stream=qstream):
        for r in range(10):
            qslaunch(r)
    qg.replay()
    qs_us = float("inf")
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        qg.replay()                      # a replay runs on the current stream: timed there
        b.record(stream)
        torch.cuda.synchronize()
        qs_us = min(qs_us, 1e3 * a.elapsed_time(b) / 10)
    del qg
    for w in qsw:
        lib.mnb_qmoe_weights_release(w)
    lib.mnb_session_destroy(qsess)
    qmoe["session_strip_major"] = {
        "path": "mnb_qmoe_weights_upload + mnb_qmoe_weights_prepack, mnb_session_run_qmoe "
                "(async session, device tensors)",
        "us": round(qs_us, 2), "GB/s": round(q_bytes / (qs_us * 1e-6) / 1e9, 1),
        "frac_hbm": round(q_bytes / (qs_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del q_w

    # The EP's Compute call (mnb_session_run, synchronous) for qkv at M=1: host I/O (A and Y in
    # pageable host memory, staged through HBM, as ORT hands them over by default) against
    # device-resident A and Y (MI355X_EP_DEVICE_MEMORY=1).  Wall clock per call, median.
    sess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(sess)))
    qk, qn = LAYER[0][1], LAYER[0][2]
    qB, qS, qZ = (t.cpu().numpy() for t in layers[0][0])
    qw = C.c_void_p()
    mnb.check(lib.mnb_weights_upload(sess, C.byref(probs[0]), qB.ctypes.data, qB.nbytes,
                                     qS.ctypes.data, qS.nbytes, qZ.ctypes.data, qZ.nbytes,
                                     C.byref(qw)))
    hA = np.ascontiguousarray(acts[0].cpu().numpy())
    hY = np.empty((1, qn), dtype=np.float16)
    dA, dY = acts[0], torch.empty(1, qn, dtype=torch.float16, device=dev)

    def io_call_us(a_ptr, a_dev, y_ptr, y_dev, reps=300):
        for _ in range(20):
            mnb.check(lib.mnb_session_run(sess, qw, 1, a_ptr, a_dev, y_ptr, y_dev))
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            mnb.check(lib.mnb_session_run(sess, qw, 1, a_ptr, a_dev, y_ptr, y_dev))
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)) * 1e6

    host_us = io_call_us(hA.ctypes.data, 0, hY.ctypes.data, 0)
    dev_us = io_call_us(dA.data_ptr(), 1, dY.data_ptr(), 1)
    torch.cuda.synchronize()
    same = bool(np.array_equal(hY.view(np.uint16), dY.cpu().numpy().view(np.uint16)))

    # Stream-aware Compute (the EP's OrtSyncStreamImpl: an async session per ORT stream): calls
    # with device tensors return once enqueued; the wall clock of `reps` calls plus the one
    # synchronisation at the end of the run, per call.
    ssess = C.c_void_p()
    mnb.check(lib.mnb_session_create(0, C.byref(ssess)))
    mnb.check(lib.mnb_session_set_async(ssess, 1))
    dY2 = torch.empty_like(dY)

    def stream_call_us(reps=300):
        for _ in range(20):
            mnb.check(lib.mnb_session_run(ssess, qw, 1, dA.data_ptr(), 1, dY2.data_ptr(), 1))
        mnb.check(lib.mnb_session_synchronize(ssess))
        t0 = time.perf_counter()
        for _ in range(reps):
            mnb.check(lib.mnb_session_run(ssess, qw, 1, dA.data_ptr(), 1, dY2.data_ptr(), 1))
        t1 = time.perf_counter()
        mnb.check(lib.mnb_session_synchronize(ssess))
        t2 = time.perf_counter()
        return (t2 - t0) / reps * 1e6, (t1 - t0) / reps * 1e6

    stream_us, enqueue_us = stream_call_us()
    same_stream = bool(np.array_equal(dY2.cpu().numpy().view(np.uint16),
                                      dY.cpu().numpy().view(np.uint16)))
    lib.mnb_session_destroy(ssess)
    lib.mnb_weights_release(qw)
    lib.mnb_session_destroy(sess)
    session_io = {"node": f"{LAYER[0][0]} M=1 K={qk} N={qn}", "host_io_us": round(host_us, 2),
                  "device_io_us": round(dev_us, 2), "outputs_identical": same,
                  "device_io_stream_us": round(stream_us, 2),
                  "device_io_stream_enqueue_us": round(enqueue_us, 2),
                  "stream_outputs_identical": same_stream,
                  "note": "host_io_us / device_io_us: median wall clock of one synchronous EP "
                          "Compute call (mnb_session_run); device_io_stream_us: stream-aware "
                          "Compute (async session, device tensors), wall clock per call over 300 "
                          "calls plus the run-end synchronisation; _enqueue_us: the calls alone"}

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    line = {
        "metric": "MatMulNBits int4 decode GB/s (% HBM peak) at M=1; prefill TFLOP/s at M=2048",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "device_ms_per_step": round(dev_ms_step, 5),
        "eager_ms_per_step": round(eager_ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 activations x int4 weights, fp32 accumulate",
        "data": "synthetic (seeded): A ~ N(0,1), uniform nibbles and zero points, scales |N(0,1)|*0.02",
        "config": {"workload": "Phi-3.5-mini decode, one token's MatMulNBits work per step: "
                               "32 layers x (qkv 3072->9216, o 3072->3072, gate_up "
                               "3072->16384, down 8192->3072), M=1, int4 block_size=32 with "
                               "zero_points, every layer its own weights",
                   "layers": LAYERS_PER_TOKEN, "launches_per_step": LAYERS_PER_TOKEN * len(LAYER),
                   "bytes_per_step": per_token, "bytes_per_layer": per_layer},
        "node_sum_ms_per_step": round(node_sum_ms, 5),
        "step_over_node_sum": round(ms_step / node_sum_ms, 4),
        "roofline": roofline,
        "per_kernel": per_kernel,
        "batched_decode": batched,
        "batched_decode_session": {
            "path": "EP session layer as the EP runs by default (ep.strip_major_weights): mnb_weights_upload + "
                    "mnb_weights_prepack (strip-major copy), mnb_session_run_device; every "
                    "node at 4-16 rows runs the batched kernel on the strip-major copy",
            "rows": batched_session},
        "prefill": prefill,
        "prefill_8bit": prefill_8bit,
        "mfma_calibration": mfma_cal,
        "accuracy_level_4": acc4,
        "decode_f32": decode_f32,
        "prefill_f32": prefill_f32,
        "moe": moe,
        "qmoe": qmoe,
        "session_io": session_io,
        "cpu_baseline": cpu,
        "stock_ort_cpu_baseline": stock_ort_probe(),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
