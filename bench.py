#!/usr/bin/env python3
"""Benchmark of the int8 QDQ path on one MI355X.

Prints ONE JSON line (driver contract). The default, --config all, runs the
five BASELINE.json configs in one process: the headline (value, roofline,
cpu_baseline) is cfg3, and `configs` holds one entry per config (cfg1, cfg2,
cfg3, cfg4, cfg5 with per-tensor weights, cfg5 with per-channel weights),
each with its own parity gate (run before its timing), value, ms_per_step,
roofline (with measured HBM traffic where a rocprofv3 summary exists) and
cpu_baseline. Single workloads (BASELINE.json configs and more):
  mobilenetv2 cfg4: MobileNetV2 int8 QDQ graph, batch 256 (depthwise VALU path
            against the pointwise MFMA GEMM); value = images/s
  bert      cfg5: BERT-base int8 encoder, 12 layers, batch 64, seq 128;
            value = sequences/s
  resnet50  cfg3 (default, the headline metric): ResNet-50 v1.5 int8 QDQ graph,
            batch 256, 224x224, run through the C++ host framework (QDQ
            fusion, NHWC layouts, HIP operators); value = images/s
  qoperator QOperator-format graph through the rest of the QLinear family
            (AveragePool, Concat, Mul, GlobalAveragePool), batch 256, 224x224;
            value = images/s, roofline = HBM of the family kernels
  qmatmul   cfg1: QLinearMatMul u8[1024,768] x i8[768,3072]; value = TOPS
  qconv     cfg2: QLinearConv 3x3 s1 p1, x u8[32,64,56,56], per-channel w
A step is one pass of the path over one batch; inputs are resident in HBM
when the timed region starts. Before timing, the GPU output is checked
bit-exact against the CPU oracle. The `roofline` object is measured live
with hipEvents on the launch stream: every node of the plan is run back to
back between two events (no event between launches, so short kernels are not
inflated), and the dominant kernel family's average launch is placed under
the roof its own algorithmic ops / bytes put it (MFMA or HBM), with each
layer's roofline fraction beside it; the `cpu_baseline` leg times a CPU
restatement on host cores on a bounded sample of the same workload.
ResNet-50 and MobileNetV2 steps run the batch as --split slices (default 2)
concurrently, one context and stream per slice (graph.SplitSession; their
graph outputs are checked bit-identical to the whole-batch context's first);
the parity gate, the per-layer table and the roofline come from the
whole-batch context, whose own step time is in config.split. BERT's
DynamicQuantizeLinear takes its scale from the whole batch, so its batch is
not split.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "int8 TOPS + % i8 MFMA peak per layer; ResNet-50-int8 images/sec b256, 1 GPU"
PEAK_I8_TOPS = 5000.0      # MI355X dense int8 MFMA, TOPS
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, GB/s


def cpu_host() -> dict:
    """The host the CPU baseline runs on: logical CPUs this process may use,
    their physical cores, the CPU model and whether AVX-512 VNNI is there."""
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except Exception:
        cpus = list(range(os.cpu_count() or 1))
    model, flags, cores = "unknown", set(), set()
    try:
        cur = {}
        for line in open("/proc/cpuinfo").read().splitlines() + [""]:
            if not line.strip():
                if cur.get("processor") is not None and int(cur["processor"]) in cpus:
                    cores.add((cur.get("physical id", "0"), cur.get("core id", cur["processor"])))
                    model = cur.get("model name", model)
                    flags = set(cur.get("flags", "").split())
                cur = {}
                continue
            k, _, v = line.partition(":")
            cur[k.strip()] = v.strip()
    except OSError:
        pass
    return {"nproc": len(cpus), "physical_cores": len(cores) or len(cpus), "cpu_model": model,
            "avx512_vnni": "avx512_vnni" in flags}


def cpu_setup():
    """Configure the oracle as the CPU baseline: conv / matmul accumulators
    through the AVX-512 VNNI restatement (oracle/nnr_vnni.c: MR 6 x NR 48
    vpdpbusd micro-kernel, weights packed once) threaded by the reference's
    int8_compute_threads over every logical CPU of this process, the rest of
    the oracle on OpenMP over the same CPUs. Falls back to the scalar
    restatement when the host has no AVX-512 VNNI, and says so. Returns
    (host description, threads, kind of kernel)."""
    from oracle import pyoracle as O
    host = cpu_host()
    O.set_threads(host["nproc"])
    O.lib().orc_set_host_threads(host["physical_cores"], host["nproc"])
    vnni = O.set_vnni(True)
    O.lib().orc_vnni_cache(1 if vnni else 0)
    host["kernels"] = ("AVX-512 VNNI restatement (vpdpbusd, MR 6 x NR 48, int8_compute_threads)" if vnni
                       else "scalar C restatement (no AVX-512 VNNI on this host)")
    return host, host["nproc"], vnni


def cpu_done():
    from oracle import pyoracle as O
    O.set_vnni(False)
    O.lib().orc_vnni_cache(0)


def timed_reps(fn, min_s, max_reps):
    """Run fn until min_s seconds or max_reps runs have passed; seconds per run."""
    fn()   # first run: packing, page faults
    t0 = time.perf_counter()
    reps = 0
    while True:
        fn()
        reps += 1
        if time.perf_counter() - t0 > min_s or reps >= max_reps:
            break
    return (time.perf_counter() - t0) / reps, reps


def cpu_seconds(args) -> float:
    """CPU-baseline time budget of one leg: --cpu-seconds (10 s for a single
    workload; the headline's in --config all, the other configs 4 s)."""
    return float(args.cpu_seconds)


def gate_images(B: int) -> list:
    """Images of a batch the parity gate compares: the first two and the
    last two, so tiles from the end of every persistent block's walk are
    checked as well as the first ones."""
    return sorted({0, min(1, B - 1), max(0, B - 2), B - 1})


def make_qconv(rng, N=32):
    import numpy as np
    x = rng.integers(0, 256, (N, 64, 56, 56), dtype=np.uint8)
    w = rng.integers(-127, 128, (64, 64, 3, 3), dtype=np.int8)
    ws = rng.uniform(0.001, 0.01, 64).astype(np.float32)
    b = rng.integers(-4096, 4097, 64).astype(np.int32)
    kw = dict(pads=(1, 1, 1, 1), y_nhwc=1, post_fn=1, x_scale=0.02, x_zp=128, w_scale=ws,
              y_scale=0.03, y_zp=0, bias=b)
    ops = 2.0 * N * 64 * 56 * 56 * 64 * 9
    # algorithmic bytes: x + y + w + per-channel params (scale f32 + bias i32)
    nbytes = N * 64 * 56 * 56 * 2 + 64 * 64 * 9 + 64 * 8
    return x, w, kw, ops, nbytes


def run_qconv(args, dev):
    import numpy as np
    import torch

    import nnr_amd as H
    from nnr_amd import _lib
    rng = np.random.default_rng(2)
    x, w, kw, ops, nbytes = make_qconv(rng)
    op = H.QLinearConv(32, 64, 56, 56, w, **kw)
    xd = torch.from_numpy(x).to(dev)
    yd = torch.empty(op.out_shape, dtype=torch.uint8, device=dev)
    # parity gate (bit-exact vs the oracle) before timing
    from oracle import pyoracle as O
    ref, br = O.Conv(32, 64, 56, 56, 64, 3, 3, **kw).run(x, w)
    op(xd, yd)
    torch.cuda.synchronize()
    assert br == op.branch and np.array_equal(yd.cpu().numpy(), ref), "parity gate failed"
    ms = time_steps(lambda: op(xd, yd), args)
    prof = profile_steps(lambda: op(xd, yd), args)
    g_launches, g_ms = prof["qgemm"]
    assert g_launches == args.steps   # one GEMM launch per step
    # the GEMM kernel's own duration: the whole step when it is the step's
    # only launch, else its event-bracketed launches
    others = sum(v[0] for k, v in prof.items() if k != "qgemm")
    kern_ms = ms if others == 0 else g_ms / g_launches
    # cpu baseline: the CPU restatement on the whole batch
    host, nthr, vnni = cpu_setup()
    oc = O.Conv(32, 64, 56, 56, 64, 3, 3, **kw)
    cpu_s, reps = timed_reps(lambda: oc.run(x, w), cpu_seconds(args), 10000)
    cpu_done()
    cpu_tops = ops / cpu_s / 1e12
    tops = ops / (ms * 1e-3) / 1e12
    rl = roofline(ops, nbytes, kern_ms, prof)
    rl["traffic"], rl["traffic_source"] = measured_traffic("qconv_cfg2_traffic.md")
    rl["counters"] = measured_counters("qconv_cfg2_counters.md")
    rl["note"] = ("achieved = the convolution's algorithmic ops and bytes / the GEMM kernel's launch time; "
                  "value = the same ops / the whole step (%d launches)" % (1 + others // args.steps))
    return dict(
        metric="QLinearConv 3x3 int8 TOPS (cfg2), 1 GPU", value=round(tops, 3), unit="TOPS", ms_per_step=ms,
        config={"workload": "cfg2 QLinearConv 3x3 s1 p1 x u8[32,64,56,56] w i8[64,64,3,3] "
                            "per-channel scales, fused Relu, NHWC out (NR16 branch, RQ-B)",
                "global_batch": 32, "branch": H.BRANCH_NAMES[op.branch]},
        parity="whole output bit-exact vs the oracle before timing",
        roofline=rl,
        cpu_baseline={"value": round(cpu_tops, 4), "unit": "TOPS", "cores": nthr, "kind": "port",
                      "sample": f"the whole batch of 32 images, mean of {reps} runs", "host": host},
        dtype="u8",
    )


def run_qmatmul(args, dev):
    """cfg1: QLinearMatMul A u8[1024,768] x B i8[768,3072] -> u8, per-tensor
    quantization (a 0.02/128, b 0.005/0, y 0.05/128), seed 1."""
    import numpy as np
    import torch

    import nnr_amd as H
    from oracle import pyoracle as O
    rng = np.random.default_rng(1)
    M, K, N = 1024, 768, 3072
    a = rng.integers(0, 256, (M, K), dtype=np.uint8)
    b = rng.integers(-127, 128, (K, N), dtype=np.int8)
    q = (0.02, 128, 0.005, 0, 0.05, 128)
    op = H.QLinearMatMul(b, q[0], q[1], q[2], q[3], q[4], q[5], m=M)
    ad = torch.from_numpy(a).to(dev)
    yd = torch.empty((M, N), dtype=torch.uint8, device=dev)
    ref = O.qlinear_matmul(a, q[0], q[1], b, q[2], q[3], q[4], q[5])
    op(ad, yd)
    torch.cuda.synchronize()
    assert np.array_equal(yd.cpu().numpy(), ref), "parity gate failed"
    ms = time_steps(lambda: op(ad, yd), args)
    prof = profile_steps(lambda: op(ad, yd), args)
    g_launches, g_ms = prof["qgemm"]
    assert g_launches == args.steps   # one kernel launch per step: its duration is ms
    ops = 2.0 * M * N * K
    nbytes = M * K + K * N + M * N
    # cpu baseline: the CPU restatement on the whole matrix
    host, nthr, vnni = cpu_setup()
    cpu_s, reps = timed_reps(lambda: O.qlinear_matmul(a, q[0], q[1], b, q[2], q[3], q[4], q[5]),
                             cpu_seconds(args), 10000)
    cpu_done()
    rl = roofline(ops, nbytes, ms, prof)
    rl["traffic"], rl["traffic_source"] = measured_traffic("qmatmul_cfg1_traffic.md")
    rl["counters"] = measured_counters("qmatmul_cfg1_counters.md")
    rl["note"] = "one launch per step: achieved = algorithmic ops and bytes / the step's time"
    return dict(
        metric="QLinearMatMul int8 TOPS (cfg1), 1 GPU", value=round(ops / (ms * 1e-3) / 1e12, 3), unit="TOPS",
        ms_per_step=ms,
        config={"workload": "cfg1 QLinearMatMul A u8[1024,768] x B i8[768,3072] -> u8 (RQ-D)",
                "global_batch": M},
        parity="whole output bit-exact vs the oracle before timing",
        roofline=rl,
        cpu_baseline={"value": round(ops / cpu_s / 1e12, 4), "unit": "TOPS", "cores": nthr,
                      "kind": "port", "sample": f"the whole 1024 x 768 x 3072 product, {reps} runs", "host": host},
        dtype="u8",
    )


def measured_traffic(name):
    """HBM bytes per launch of the dominant kernel, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE passes summarized under profiles/ (copy-kernel
    calibrated); None when no summary exists for this workload."""
    import re
    if not name:
        return None, None
    path = os.path.join(ROOT, "profiles", name)
    try:
        txt = open(path).read()
    except OSError:
        return None, None
    m = re.search(r"^hbm_bytes_per_launch: (\d+)$", txt, re.M)
    return (int(m.group(1)), "profiles/" + name) if m else (None, None)


def time_steps(fn, args) -> float:
    import torch
    for _ in range(args.warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / args.steps


def profile_steps(fn, args) -> dict:
    """Per-kernel launch times over K steps (hipEvents around each launch)."""
    import torch
    from nnr_amd import _lib
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(args.steps):
        fn()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    out = _lib.profile_read()
    _lib.profile_reset()
    return out


def roofline(ops, nbytes, kern_ms, prof, kernel="qgemm_dma_kernel"):
    """Roofline object of the dominant kernel: one average launch does `ops`
    algorithmic int8 ops and moves `nbytes` algorithmic bytes in `kern_ms`.
    `bound` is the roof its own model puts it under -- MFMA when ops / peak
    exceeds bytes / HBM peak, else HBM -- and `achieved` / `frac` are on that
    roof; the other roof's fraction is reported beside it."""
    t_mfma = ops / (PEAK_I8_TOPS * 1e12)
    t_hbm = nbytes / (PEAK_HBM_GBS * 1e9)
    tops = ops / (kern_ms * 1e-3) / 1e12
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    bound = "mfma" if t_mfma >= t_hbm else "hbm"
    r = {"kernel": kernel, "bound": bound,
         "achieved": round(tops if bound == "mfma" else gbs, 2),
         "peak": PEAK_I8_TOPS if bound == "mfma" else PEAK_HBM_GBS,
         "unit": "TOPS" if bound == "mfma" else "GB/s",
         "frac": round((tops / PEAK_I8_TOPS) if bound == "mfma" else (gbs / PEAK_HBM_GBS), 4),
         "traffic": None, "avg_launch_ms": round(kern_ms, 5),
         "alg_ops_per_launch": ops, "alg_bytes_per_launch": nbytes,
         "mfma": {"achieved_tops": round(tops, 1), "frac": round(tops / PEAK_I8_TOPS, 4)},
         "hbm": {"achieved_gbs": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)},
         "launches": {k: {"n": v[0], "avg_ms": round(v[1] / max(1, v[0]), 5)}
                      for k, v in prof.items()}}
    return r


def node_rows(s, args, reps=10):
    """Per-node rows of the executed plan: device time of each node run
    `reps` times back to back (no event between launches), its algorithmic
    ops and bytes, and the roofline each is under: t_roof = max(ops / i8
    peak, bytes / HBM peak), roof_frac = t_roof / measured."""
    from nnr_amd import _lib
    rows = []
    prof = s.profile()
    for i, p in enumerate(prof):
        # kernel launches of this node (one run under the launch profiler)
        _lib.profile_reset()
        _lib.profile_enable(True)
        s.time_node(i, 1)
        _lib.profile_enable(False)
        launches = sum(v[0] for v in _lib.profile_read().values())
        _lib.profile_reset()
        t = s.time_node(i, reps)
        t_mfma = p["ops"] / (PEAK_I8_TOPS * 1e12) * 1e3
        t_hbm = p["bytes"] / (PEAK_HBM_GBS * 1e9) * 1e3
        rows.append(dict(name=p["name"], op=p["op"], variant=p["variant"], ms=t, ops=p["ops"], launches=launches,
                         bytes=p["bytes"], t_roof_ms=max(t_mfma, t_hbm),
                         bound="mfma" if t_mfma >= t_hbm and p["ops"] else "hbm"))
    return rows


def family_roofline(rows, select, kprof, extra_ms=0.0, extra_launches=0, kernel="qgemm_dma_kernel"):
    """Roofline of a kernel family over one step: the selected nodes (one
    launch of the family each; `extra_ms` of other kernels inside them is
    taken out), plus the per-layer aggregate sum(t_roof) / sum(measured)."""
    sel = [r for r in rows if select(r)]
    n = len(sel) + extra_launches
    fam_ms = sum(r["ms"] for r in sel) - extra_ms
    ops = sum(r["ops"] for r in sel)
    nbytes = sum(r["bytes"] for r in sel)
    rl = roofline(ops / n, nbytes / n, fam_ms / n, kprof, kernel=kernel)
    rl["per_layer"] = {"roof_ms": round(sum(r["t_roof_ms"] for r in sel), 4),
                       "measured_ms": round(sum(r["ms"] for r in sel), 4),
                       "roofline_time_frac": round(sum(r["t_roof_ms"] for r in sel) /
                                                   max(1e-9, sum(r["ms"] for r in sel)), 4),
                       "layers_mfma_bound": sum(1 for r in sel if r["bound"] == "mfma"),
                       "layers_hbm_bound": sum(1 for r in sel if r["bound"] == "hbm")}
    return rl, fam_ms


def measured_counters(name):
    """MFMA / LDS counter figures of the dominant kernel from a rocprofv3
    --pmc summary under profiles/ (lines `key: value`), or None."""
    import re
    path = os.path.join(ROOT, "profiles", name)
    try:
        txt = open(path).read()
    except OSError:
        return None
    out = {}
    for k in ("mfma_util_pct", "mfma_i8_ops_executed_per_step", "lds_bank_conflict_pct", "lds_util_pct"):
        m = re.search(r"^%s: ([0-9.eE+-]+)$" % k, txt, re.M)
        if m:
            out[k] = float(m.group(1))
    if out:
        out["source"] = "profiles/" + name
    return out or None


def planned_session(args, g, feeds, ref):
    """The context that is timed. With --memory-planning 1 (the default) it
    shares device memory between intermediates (one arena: lifetime slots,
    in-place outputs, concat parts inside their output); its graph outputs
    must equal, bit for bit, those of the unplanned context `ref` whose every
    intermediate tensor the parity gate checked. Returns (session, memory
    report)."""
    import numpy as np
    import torch

    from nnr_amd import graph as G
    mem = {"planned": bool(args.memory_planning), "device_bytes_unplanned": ref.device_bytes()}
    if not args.memory_planning and not args.onnx:
        mem["device_bytes"] = ref.device_bytes()
        return ref, mem
    if args.onnx:
        # the model as an ONNX file (initializers in external data, symbolic
        # batch), loaded by the C++ loader
        import tempfile

        from nnr_amd import onnx_io
        d = tempfile.mkdtemp(prefix="nnr_onnx_")
        path = os.path.join(d, "model.onnx")
        onnx_io.save(g, path, external_data=True, sym_dims=(0,))
        t0 = time.perf_counter()
        s = G.Session(None, onnx=path, sym_dim=next(iter(feeds.values())).shape[0],
                      memory_planning=bool(args.memory_planning))
        mem["onnx"] = {"model_bytes": os.path.getsize(path), "external_bytes": os.path.getsize(path + ".data"),
                       "load_and_prepare_ms": round((time.perf_counter() - t0) * 1e3, 1)}
    else:
        s = G.Session(g, memory_planning=True)
    for k, v in feeds.items():
        s.set_input(k, v)
    s.run()
    torch.cuda.synchronize()
    for o in g.outputs:
        assert np.array_equal(s.output(o)[0], ref.output(o)[0]), f"planned context differs at {o}"
    if not args.memory_planning:
        mem["device_bytes"] = s.device_bytes()
        return s, mem
    stats, _ = s.memory_plan()
    mem.update(device_bytes=s.device_bytes(), arena_bytes=stats["pool_bytes"],
               pooled_tensors=stats["intermediates"], slots=stats["slots"], inplace=stats["inplace"],
               concat_parts=stats["concat"])
    return s, mem


def layer_table(rows, args) -> list:
    """Per-layer rows (each node timed back to back): TOPS and % of the i8
    MFMA peak for operators with algorithmic ops, GB/s and % of HBM peak for
    all, and the fraction of its own roofline (max of the two times); to
    stderr and optionally to --layers-out."""
    layers = []
    for r in rows:
        t = r["ms"]
        row = {"name": r["name"], "op": r["op"], "branch": r["variant"], "ms": round(t, 4),
               "launches": r["launches"]}
        if r["ops"]:
            row["tops"] = round(r["ops"] / (t * 1e-3) / 1e12, 1)
            row["pct_i8_peak"] = round(100 * row["tops"] / PEAK_I8_TOPS, 2)
        row["gbs"] = round(r["bytes"] / (t * 1e-3) / 1e9, 1)
        row["pct_hbm"] = round(100 * row["gbs"] / PEAK_HBM_GBS, 2)
        row["bound"] = r["bound"]
        row["pct_roofline"] = round(100 * r["t_roof_ms"] / t, 1)
        layers.append(row)
    if args.layers_out:
        with open(args.layers_out, "w") as f:
            json.dump(layers, f, indent=1)
    for row in layers:
        print(json.dumps(row), file=sys.stderr)
    return layers


WORKLOADS = {
    "resnet50": "cfg3 ResNet-50 v1.5 int8 QDQ, batch {B}, 224x224 (53 QLinearConv, 16 QLinearAdd, "
                "uint8 MaxPool, fp32 GAP+FC)",
    "mobilenetv2": "cfg4 MobileNetV2 int8 QDQ, batch {B}, 224x224 (52 QLinearConv incl. 17 "
                   "depthwise, 10 QLinearAdd, ReLU6 in the quantization range, fp32 GAP+FC)",
}


def split_steps(args, make_graph, B, feeds, ref, outputs):
    """The batch as args.split slices run concurrently (graph.SplitSession:
    one context and stream per slice, one group step on the current stream).
    Every image's computation is independent of the others' in these
    graphs, so the graph outputs must equal the whole-batch context's bit
    for bit; then the timed steps."""
    import numpy as np
    import torch
    from nnr_amd import graph as G
    ss = G.SplitSession(make_graph, batch=B, parts=args.split, memory_planning=bool(args.memory_planning))
    try:
        for k, v in feeds.items():
            ss.set_input(k, v)
        ss.run()
        torch.cuda.synchronize()
        for o in outputs:
            assert np.array_equal(ss.output(o)[0], ref.output(o)[0]), f"split plan differs at {o}"
        ms = time_steps(ss.run, args)
        info = {"parts": args.split, "images_per_part": B // args.split, "hip_graph": ss.graph_active(),
                "device_bytes": ss.device_bytes()}
    finally:
        ss.close()
    return ms, info


def run_model(args, dev, model):
    import numpy as np
    import torch

    from nnr_amd import _lib, graph as G, synth
    from oracle import graph_oracle
    from oracle import pyoracle as O

    B = args.batch
    make_graph = lambda b: {"resnet50": synth.resnet50, "mobilenetv2": synth.mobilenetv2}[model](batch=b, hw=224)
    g = make_graph(B)
    rng = np.random.default_rng(10)
    x = rng.random((B, 3, 224, 224), dtype=np.float32)
    s = G.Session(g)
    s.set_input("input", x)
    s.run()
    torch.cuda.synchronize()
    plan = s.plan()
    fmt = lambda n: s.tensor_info(n)[3]
    # parity gate: the oracle replays the plan on the first two and the last
    # two images of the batch; every int8 tensor of the plan must match
    idx = gate_images(B)
    env = graph_oracle.run_plan(plan, g, {"input": x[idx]}, fmt)
    n_int = 0
    for p in plan:
        o = p["outputs"][0]
        dev_t, _ = s.output(o)
        if dev_t.dtype in (np.uint8, np.int8):
            assert np.array_equal(dev_t[idx], env[o]), f"parity gate failed at {p['name']}"
            n_int += 1
        else:
            assert np.allclose(dev_t[idx], env[o], atol=1e-3, rtol=1e-4), p["name"]
        del dev_t
    parity = (f"oracle replay of the plan on images {idx} of {B}: all {n_int} int8 tensors bit-exact, "
              "fp32 within 1e-3")
    s, mem = planned_session(args, g, {"input": x}, s)
    ms = time_steps(s.run, args)
    mem["hip_graph"] = s.graph_active()
    split = None
    if args.split > 1 and not args.onnx and B % args.split == 0:
        split_ms, split = split_steps(args, make_graph, B, {"input": x}, s, g.outputs)
        split["one_context_ms_per_step"] = round(ms, 5)
        split["one_context_value"] = round(B / (ms * 1e-3), 1)
        parity += (f"; the batch as {args.split} concurrent slices gives the whole-batch context's "
                   "graph outputs bit for bit")
    # per-kernel launch times (an event pair around every launch) and
    # per-node times (each node run back to back, no event between launches)
    kprof = profile_steps(s.run, args)
    rows = node_rows(s, args)
    layer_table(rows, args)
    conv_ops = sum(r["ops"] for r in rows if r["op"] == "QLinearConv")
    # the conv GEMM kernel, with or without a fused residual add: one launch
    # per QLinearConv node; the first layer's node also runs its input
    # layout kernel, and a conv on channels that are not a multiple of 16 a
    # channel-padding kernel (timed by the launch profiler), taken out here
    copies_ms = 0.0
    for k in ("quantize_first_layer_copies", "first_layer_copies", "pad_channels_u8", "nchw_to_nhwc_u8"):
        if k in kprof:
            copies_ms += kprof[k][1] / args.steps
    is_conv = lambda r: r["op"] == "QLinearConv" and r["variant"] != "DW"
    rl, fam_ms = family_roofline(rows, is_conv, kprof, extra_ms=copies_ms)
    rl["kernel"] = "qgemm_dma_kernel / qgemm_direct_kernel / stem_conv_kernel (conv GEMM family)"
    rl["traffic"], rl["traffic_source"] = measured_traffic(
        f"{model}_b256_conv_gemm_traffic.md" if B == 256 else None)
    rl["counters"] = measured_counters(f"{model}_b256_conv_gemm_counters.md") if B == 256 else None
    g_launches = sum(kprof[k][0] for k in ("qgemm", "qgemm_add") if k in kprof)
    g_ms = sum(kprof[k][1] for k in ("qgemm", "qgemm_add") if k in kprof)
    rl["event_per_launch_avg_ms"] = round(g_ms / max(1, g_launches), 5)
    n_fused = s.fusion_stat("conv_add")
    n_conv = sum(1 for r in rows if is_conv(r))
    rl["note"] = (f"one average launch of the {n_conv} conv GEMM launches of a step ({n_fused} with the "
                  "residual add fused): algorithmic ops and bytes / kernel time, each node timed back to "
                  "back with no event between launches (the first layer's input-layout kernel taken "
                  "out); bound = the roof its ops / bytes put it under; per_layer = sum of each layer's "
                  "max(ops / MFMA peak, bytes / HBM peak) over the sum of measured times")
    qgemm_ms_per_step = fam_ms
    if "depthwise" in kprof:
        # the depthwise convolutions are HBM-bound: their own roofline
        dw_rows = [r for r in rows if r["op"] == "QLinearConv" and r["variant"] == "DW"]
        dw_ms = sum(r["ms"] for r in dw_rows)
        dw_bytes = sum(r["bytes"] for r in dw_rows)
        dw_gbs = dw_bytes / (dw_ms * 1e-3) / 1e9
        rl["depthwise"] = {"bound": "hbm", "achieved": round(dw_gbs, 1), "peak": PEAK_HBM_GBS,
                           "unit": "GB/s", "frac": round(dw_gbs / PEAK_HBM_GBS, 4),
                           "launches_per_step": len(dw_rows), "alg_bytes_per_step": dw_bytes,
                           "avg_launch_ms": round(dw_ms / max(1, len(dw_rows)), 5)}
    # cpu baseline: the CPU restatement replays the same plan on 8 images
    host, nthr, vnni = cpu_setup()
    ns = min(8, B)
    cpu_s, reps = timed_reps(lambda: graph_oracle.run_plan(plan, g, {"input": x[:ns]}, fmt), cpu_seconds(args), 100)
    cpu_done()
    cpu_img_s = ns / cpu_s
    step_ms = split_ms if split else ms
    imgs = B / (step_ms * 1e-3)
    return dict(
        metric=METRIC if model == "resnet50" else "MobileNetV2-int8 images/sec b256 (cfg4), 1 GPU",
        value=round(imgs, 1), unit="images/s", ms_per_step=step_ms,
        config={"workload": WORKLOADS[model].format(B=B), "global_batch": B, "split": split,
                "branches": {b: sum(1 for p in plan if p["variant"].split("+")[0] == b)
                             for b in ("FIRST", "DW", "NR16", "PACKED")},
                "adds_fused_into_conv": s.fusion_stat("conv_add"),
                "conv_gemm_tops": round(sum(r["ops"] for r in rows if is_conv(r)) /
                                        (qgemm_ms_per_step * 1e-3) / 1e12, 1),
                "memory": mem},
        parity=parity,
        roofline=rl,
        cpu_baseline={"value": round(cpu_img_s, 3), "unit": "images/s", "cores": nthr,
                      "kind": "port", "sample": f"replay of the executed plan on {ns} of the {B} images, "
                                                f"{reps} runs", "host": host},
        dtype="u8",
    )


def run_bert(args, dev):
    """cfg5: BERT-base int8 encoder, 12 layers, batch 64, seq 128."""
    import numpy as np
    import torch

    from nnr_amd import graph as G, synth
    from oracle import graph_oracle
    from oracle import pyoracle as O

    B = 64 if args.batch == 256 else args.batch
    S, L = 128, 12
    pc = bool(args.per_channel)
    g = synth.bert(batch=B, seq=S, layers=L, per_channel=pc)
    proj = "MatMulInteger" if pc else "QLinearMatMul"
    rng = np.random.default_rng(20)
    x = rng.uniform(-1.0, 1.0, (B, S, 768)).astype(np.float32)
    s = G.Session(g)
    s.set_input("input", x)
    s.run()
    torch.cuda.synchronize()
    plan = s.plan()
    fmt = lambda n: s.tensor_info(n)[3]
    # parity gate: every projection (QLinearMatMul, or MatMulInteger with its
    # fused Cast / scale / bias chain) of the first layer, recomputed by the
    # oracle from the device's own inputs (dynamic scale / zero point
    # included) on the first two sequences
    idx = gate_images(B)

    def dev_slice(name):
        t, _ = s.output(name)
        return t[idx] if t.ndim >= 1 and t.shape[0] == B else t

    skip = {p["op"] for p in plan} - {proj}
    env = graph_oracle.run_plan(plan, g, {}, fmt, source=dev_slice, skip_ops=skip,
                                stop_after="l0_ffn2", keep_chain=True)
    checked = 0
    for p in plan:
        if p["op"] == proj and p["outputs"][0] in env:
            d, ref = dev_slice(p["outputs"][0]), env[p["outputs"][0]]
            if p["variant"].endswith("+Codes"):
                # the chain stores its uint8 QLinearMatMul bytes for the
                # DynamicQuantizeLinear after it
                ref = env[g.node_by_name(p["fused_chain"][0]).inputs[0]]
                assert np.array_equal(d, ref), f"parity gate failed at {p['name']}"
            elif any(g.node_by_name(c).op == "Gelu" for c in p.get("fused_chain") or []):
                # erf in float64 against the device's fp32 erff: a few ulps
                assert np.allclose(d, ref, rtol=2e-6, atol=1e-7), f"parity gate failed at {p['name']}"
            else:
                assert np.array_equal(d, ref), f"parity gate failed at {p['name']}"
            checked += 1
    assert checked == 6
    parity = (f"the first layer's {checked} {proj} projections recomputed by the oracle from the device's own "
              f"inputs on sequences {idx} of {B}: bit-exact (an fp32 Gelu chain end within 2e-6)")
    readers = [p for p in plan if "Codes" in p["variant"] and p["op"] != proj]
    if readers:
        # the operators that form their input from stored chain bytes
        # (DynamicQuantizeLinear after FF1, the attention, the LayerNorms)
        # and every quantizer and the graph output, against a context that
        # materializes the fp32 tensors (whose operators the per-node tests
        # check): every layer, the whole batch
        ref_s = G.Session(g, codes=False)
        ref_s.set_input("input", x)
        ref_s.run()
        cmp = [p for p in plan if p["op"] in ("DynamicQuantizeLinear", "MultiHeadAttention", "LayerNormalization")]
        n = 0
        for p in cmp:
            for o in p["outputs"]:
                if not o or s.tensor_info(o)[1] != ref_s.tensor_info(o)[1]:
                    continue
                a, b = np.atleast_1d(s.output(o)[0]), np.atleast_1d(ref_s.output(o)[0])
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"parity gate failed at {p['name']}"
                n += 1
        for o in g.outputs:
            assert np.array_equal(s.output(o)[0].view(np.uint8), ref_s.output(o)[0].view(np.uint8)), \
                "parity gate failed at the graph output"
        del ref_s
        parity += (f"; with the projections storing uint8 bytes that {len(readers)} readers turn back into "
                   f"values, the outputs of every quantizer, attention and LayerNorm ({n} tensors) and the "
                   f"graph output equal, bit for bit over the whole batch, a context that materializes the "
                   f"fp32 projection outputs")
    s, mem = planned_session(args, g, {"input": x}, s)
    ms = time_steps(s.run, args)
    mem["hip_graph"] = s.graph_active()
    kprof = profile_steps(s.run, args)
    rows = node_rows(s, args)
    layer_table(rows, args)
    is_mm = lambda r: r["op"] == proj
    # the members of a grouped Q / K / V launch run inside their leader's
    # launch: their work counts, their (empty) launches do not
    grouped = sum(1 for r in rows if is_mm(r) and "(grouped)" in r["variant"])
    rl, mm_ms = family_roofline(rows, is_mm, kprof, extra_launches=-grouped)
    mm_ops = sum(r["ops"] for r in rows if is_mm(r))
    rl["kernel"] = f"qgemm_dma_kernel ({proj} family)"
    tag = "bert_b64_s128_pc" if pc else "bert_b64_s128"
    rl["traffic"], rl["traffic_source"] = measured_traffic(f"{tag}_matmul_traffic.md" if B == 64 else None)
    rl["counters"] = measured_counters(f"{tag}_matmul_counters.md") if B == 64 else None
    g_launches, g_ms = kprof["qgemm"]
    rl["event_per_launch_avg_ms"] = round(g_ms / max(1, g_launches), 5)
    rl["note"] = (f"one average launch of the {round(g_launches / args.steps)} {proj} launches of one "
                  "step: algorithmic ops and bytes / kernel time, each node timed back to back with no "
                  "event between launches")
    # cpu baseline: the CPU restatement replays an 8-sequence copy of the graph
    ns = min(8, B)
    g1 = synth.bert(batch=ns, seq=S, layers=L, per_channel=pc)
    plan1 = G.Session(g1, device=False).plan()
    host, nthr, vnni = cpu_setup()
    cpu_s, reps = timed_reps(lambda: graph_oracle.run_plan(plan1, g1, {"input": x[:ns]}, lambda n: 0),
                             cpu_seconds(args), 50)
    cpu_done()
    cpu_seq_s = ns / cpu_s
    return dict(
        metric="BERT-base int8 encoder sequences/sec (12 layers, B64, S128), 1 GPU",
        value=round(B / (ms * 1e-3), 1), unit="sequences/s", ms_per_step=ms,
        config={"workload": f"cfg5 BERT-base int8, 12 layers, hidden 768, 12 heads, FFN 3072, "
                            f"seq {S}, batch {B} (72 projections on DynamicQuantizeLinear activations, "
                            + ("per-channel int8 weights: MatMulInteger -> Cast -> Mul(x_scale * w_scale[N]) "
                               "-> Add" if pc else "per-tensor int8 weights: QLinearMatMul") +
                            "; fp32 attention, Softmax, LayerNorm, Gelu)",
                "global_batch": B, "seq_len": S, "weights": "per-channel" if pc else "per-tensor",
                "int8_tops": round(mm_ops / (mm_ms * 1e-3) / 1e12, 1), "memory": mem},
        parity=parity,
        roofline=rl,
        cpu_baseline={"value": round(cpu_seq_s, 3), "unit": "sequences/s", "cores": nthr,
                      "kind": "port", "sample": f"replay of the plan on {ns} sequences, {reps} runs "
                                                "(int8 GEMMs in the restatement, fp32 glue in numpy)",
                      "host": host},
        dtype="u8",
    )


# QLinear-family operators of the QOperator graph and the launch-profiler
# name of the kernel each one runs
QFAMILY = {"QLinearMul": "qlinear_mul", "QLinearAveragePool": "qlinear_avgpool",
           "QLinearConcat": "qlinear_concat", "QLinearGlobalAveragePool": "qlinear_global_avgpool"}


def run_bn(args, dev):
    """fold_bn_qdq's two patterns at batch 256: Q -> QLinearConv 3x3 (64 -> 64,
    NHWC) -> DQ -> BN -> Q -> DQ and the fp32 input -> BN -> Q -> DQ, 56x56.
    The roofline is the folded BatchNormalization kernel's (HBM)."""
    return run_qoperator(args, dev, graph="bn")


def run_qoperator(args, dev, graph="qoperator"):
    """QOperator-format graph (quantized operators instead of QDQ pairs):
    QLinearConv -> QLinearAveragePool -> two QLinearConv branches ->
    QLinearConcat -> QLinearMul (per channel, then squared) ->
    QLinearGlobalAveragePool, batch 256 at 224x224. The roofline is the
    HBM one of the QLinear-family kernel that takes the most time per step;
    every family kernel is listed with its own achieved GB/s."""
    import numpy as np
    import torch

    from nnr_amd import graph as G, synth
    from oracle import graph_oracle
    from oracle import pyoracle as O

    B = args.batch
    if graph == "bn":
        HW, Cin = 56, 64
        g = synth.bn_net(batch=B, C=Cin, hw=HW)
        family_ops = {"BatchNormalization": "batchnorm_u8"}
    else:
        HW, Cin = 224, 3
        g = synth.qoperator_net(batch=B, hw=HW)
        family_ops = QFAMILY
    rng = np.random.default_rng(24)
    x = rng.uniform(-1.0, 1.5, (B, Cin, HW, HW)).astype(np.float32)
    s = G.Session(g)
    s.set_input("input", x)
    s.run()
    torch.cuda.synchronize()
    plan = s.plan()
    fmt = lambda n: s.tensor_info(n)[3]
    # parity gate: the oracle replays the plan on the first images
    ng = 2
    env = graph_oracle.run_plan(plan, g, {"input": x[:ng]}, fmt)
    for p in plan:
        o = p["outputs"][0]
        dev_t, _ = s.output(o)
        if dev_t.dtype in (np.uint8, np.int8):
            assert np.array_equal(dev_t[:ng], env[o]), f"parity gate failed at {p['name']}"
        else:
            assert np.allclose(dev_t[:ng], env[o], atol=1e-3, rtol=1e-4), p["name"]
    s, mem = planned_session(args, g, {"input": x}, s)
    ms = time_steps(s.run, args)
    mem["hip_graph"] = s.graph_active()
    kprof = profile_steps(s.run, args)
    rows = node_rows(s, args)
    layer_table(rows, args)
    family = {}
    for op, kern in family_ops.items():
        if kern not in kprof:
            continue
        n, _ = kprof[kern]
        sel = [r for r in rows if r["op"] == op]
        nbytes = sum(r["bytes"] for r in sel)   # per run = per step
        kms = sum(r["ms"] for r in sel) * args.steps   # back-to-back node times
        gbs = nbytes / (kms / args.steps * 1e-3) / 1e9
        family[kern] = {"op": op, "achieved": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                        "launches_per_step": round(n / args.steps), "alg_bytes_per_step": nbytes,
                        "avg_launch_ms": round(kms / n, 5), "ms_per_step": round(kms / args.steps, 5)}
    assert len(family) == len(family_ops), sorted(family)
    top = max(family, key=lambda k: family[k]["ms_per_step"])
    f = family[top]
    rl = {"kernel": top, "bound": "hbm", "achieved": f["achieved"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
          "frac": f["frac"], "traffic": None, "avg_launch_ms": f["avg_launch_ms"],
          "alg_bytes_per_launch": f["alg_bytes_per_step"] / f["launches_per_step"],
          "family": family,
          "launches": {k: {"n": v[0], "avg_ms": round(v[1] / max(1, v[0]), 5)} for k, v in kprof.items()},
          "note": "achieved = algorithmic bytes (inputs read once + output written) of the operator's "
                  "launches in one step / their kernel time (each node timed back to back, no event "
                  "between launches)"}
    host, nthr, vnni = cpu_setup()
    ns = min(8, B)
    cpu_s, reps = timed_reps(lambda: graph_oracle.run_plan(plan, g, {"input": x[:ns]}, fmt), cpu_seconds(args), 100)
    cpu_done()
    cpu_img_s = ns / cpu_s
    if graph == "bn":
        metric = "DQ->BN->Q / BN->Q folded graph images/sec b256 (fold_bn_qdq), 1 GPU"
        workload = (f"batch {B}, 64x{HW}x{HW}: Q -> QLinearConv 3x3 64->64 (NHWC) -> DQ -> BatchNormalization -> "
                    "Q -> DQ, and fp32 input -> BatchNormalization -> Q -> DQ (NCHW); both BNs folded to "
                    "per-channel uint8 affines")
    else:
        metric = ("QOperator-format int8 graph images/sec b256 (QLinearConv, QLinearAveragePool, "
                  "QLinearConcat, QLinearMul, QLinearGlobalAveragePool), 1 GPU")
        workload = (f"QOperator graph, batch {B}, {HW}x{HW}: QLinearConv 3x3 (3->16), QLinearAveragePool 3x3/2 "
                    "pad 1, QLinearConv 1x1 (16->24) and 3x3 (16->8), QLinearConcat (24+8, one part copied), "
                    "QLinearMul by a per-channel constant and by itself, QLinearGlobalAveragePool")
    return dict(
        metric=metric,
        value=round(B / (ms * 1e-3), 1), unit="images/s", ms_per_step=ms,
        config={"workload": workload,
                "global_batch": B, "memory": mem,
                "ops": [p["op"] + (":" + p["variant"] if p["variant"] else "") for p in plan]},
        roofline=rl,
        cpu_baseline={"value": round(cpu_img_s, 3), "unit": "images/s", "cores": nthr, "kind": "port",
                      "sample": f"replay of the plan on {ns} of the {B} images, {reps} runs", "host": host},
        dtype="u8",
    )


def run_convinteger(args, dev):
    """ConvInteger at cfg2's shape: x u8[32,64,56,56], w i8[64,64,3,3], pad 1,
    per-channel weight zero points; int32 output. NHWC copy of the input,
    per-call weight packing and per-pixel patch sums, then the implicit-GEMM
    i8 MFMA kernel whose epilogue adds the weight zero-point term and stores
    int32 NCHW; value = TOPS of the whole operator."""
    import ctypes as C

    import numpy as np
    import torch

    import nnr_amd as H
    from nnr_amd import _lib
    from oracle import pyoracle as O
    L = _lib.lib()
    N, Cc, HW, OC = 32, 64, 56, 64
    rng = np.random.default_rng(32)
    x = rng.integers(0, 256, (N, Cc, HW, HW), dtype=np.uint8)
    w = rng.integers(-128, 128, (OC, Cc, 3, 3), dtype=np.int8)
    wz = rng.integers(-8, 8, OC).astype(np.int32)
    xd, wd = torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)
    wzd = torch.from_numpy(wz).to(dev)
    y = torch.empty((N, OC, HW, HW), dtype=torch.int32, device=dev)
    h = C.c_void_p()
    _lib.check(L.nnrh_conv_integer_create(C.byref(h), N, Cc, HW, HW, OC, 3, 3, 1, 1, 1, 1, 1, 1, HW, HW, 1,
                                          H.U8, H.S8))
    st = _lib.cur_stream()

    def step():
        _lib.check(L.nnrh_conv_integer_run(h, _lib.ptr(xd), _lib.ptr(wd), 117, 0, _lib.ptr(wzd), _lib.ptr(y), st))

    step()
    torch.cuda.synchronize()
    ref = O.conv_integer(x[:2], w, 117, wz, pads=(1, 1))
    assert np.array_equal(y[:2].cpu().numpy(), ref), "parity gate failed"
    ms = time_steps(step, args)
    kprof = profile_steps(step, args)
    L.nnrh_conv_integer_destroy(h)
    ops = 2.0 * N * OC * HW * HW * Cc * 9
    nbytes = x.nbytes + w.nbytes + N * OC * HW * HW * 4
    g_launches, g_ms = kprof["qgemm"]
    rl = roofline(ops / (g_launches / args.steps), nbytes, g_ms / g_launches, kprof)
    rl["traffic"] = None
    rl["note"] = ("achieved = algorithmic ops of the convolution / the GEMM kernel's time; value = the same ops / "
                  "the whole operator (NHWC copy, weight packing, patch sums, GEMM)")
    host, nthr, vnni = cpu_setup()
    cpu_s, reps = timed_reps(lambda: O.conv_integer(x, w, 117, wz, pads=(1, 1)), cpu_seconds(args), 1000)
    cpu_done()
    return dict(metric="ConvInteger int8 TOPS (cfg2 shape: u8[32,64,56,56] x i8[64,64,3,3], pad 1), 1 GPU",
                value=round(ops / (ms * 1e-3) / 1e12, 1), unit="TOPS", ms_per_step=ms,
                config={"workload": "ConvInteger 3x3 s1 p1, x u8[32,64,56,56], w i8[64,64,3,3], per-channel "
                                    "w_zero_point, int32 output", "global_batch": N},
                roofline=rl,
                cpu_baseline={"value": round(ops / cpu_s / 1e12, 4), "unit": "TOPS", "cores": nthr,
                              "kind": "port", "sample": f"the whole batch of 32 images, mean of {reps} runs",
                              "host": host},
                dtype="u8")


def run_hbm_copy(args, dev):
    """Device-to-device copy of a known size through hipMemcpyAsync: the
    calibration kernel for the FETCH_SIZE / WRITE_SIZE counters and the
    achievable-HBM reference for the roofline."""
    import torch

    from nnr_amd import _lib
    L = _lib.lib()
    nbytes = 1 << 30
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(7)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    st = _lib.cur_stream()

    def step():
        _lib.check(L.nnrh_memcpy(_lib.ptr(dst), _lib.ptr(src), nbytes, 2, st))

    ms = time_steps(step, args)
    gbs = 2 * nbytes / (ms * 1e-3) / 1e9
    return dict(metric="HBM device-to-device copy (read + write bytes / s)", value=round(gbs, 1),
                unit="GB/s", ms_per_step=ms,
                config={"workload": "hipMemcpyAsync D2D, 1 GiB", "bytes_per_copy": nbytes},
                roofline={"kernel": "copy", "bound": "hbm", "achieved": round(gbs, 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": 2 * nbytes},
                cpu_baseline=None, dtype="u8")


# the five BASELINE.json configs of --config all: key, workload runner, the
# arguments it runs with (cfg5 in both weight forms)
ALL_CONFIGS = (
    ("cfg1", "qmatmul", {}),
    ("cfg2", "qconv", {}),
    ("cfg4", "mobilenetv2", {}),
    ("cfg5", "bert", {"per_channel": 0}),
    ("cfg5_per_channel", "bert", {"per_channel": 1}),
)
CONFIG_KEYS = ("metric", "value", "unit", "ms_per_step", "parity", "roofline", "cpu_baseline", "dtype")


def release_device():
    """Free what the finished leg held on the device before the next one."""
    import gc

    import torch
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def run_all(args, dev, runners):
    """cfg3 (the headline) and then cfg1, cfg2, cfg4, cfg5 (per-tensor and
    per-channel weights) in one process, each leg gated, timed and profiled
    on its own; the CPU baseline of the headline takes --cpu-seconds, the
    others --cpu-seconds-other."""
    import copy
    t0 = time.perf_counter()
    print("[bench] cfg3 resnet50", file=sys.stderr, flush=True)
    head = runners["resnet50"](args, dev)
    configs = {"cfg3": {k: head.get(k) for k in CONFIG_KEYS}}
    configs["cfg3"]["workload"] = head["config"]["workload"]
    for key, name, extra in ALL_CONFIGS:
        release_device()
        a = copy.copy(args)
        a.cpu_seconds = args.cpu_seconds_other
        a.layers_out = None
        for k, v in extra.items():
            setattr(a, k, v)
        print(f"[bench] {key} {name} {extra}", file=sys.stderr, flush=True)
        t1 = time.perf_counter()
        r = runners[name](a, dev)
        c = {k: r.get(k) for k in CONFIG_KEYS}
        c["workload"] = r["config"]["workload"]
        c["leg_s"] = round(time.perf_counter() - t1, 1)
        configs[key] = c
    head["configs"] = configs
    head["config"]["all_configs_wall_s"] = round(time.perf_counter() - t0, 1)
    return head


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="all",
                    choices=["all", "resnet50", "mobilenetv2", "bert", "qoperator", "bn", "convinteger", "qconv",
                             "qmatmul", "hbm_copy"],
                    help="all (default): the five BASELINE configs, cfg3 as the headline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="time budget of the CPU-baseline leg (the headline's with --config all)")
    ap.add_argument("--cpu-seconds-other", type=float, default=4.0,
                    help="--config all: CPU-baseline budget of the configs other than cfg3")
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--layers-out", default=None, help="write the per-layer table (JSON) here")
    ap.add_argument("--onnx", type=int, default=0, choices=[0, 1],
                    help="graph configs: time the model written as an ONNX file and loaded by the C++ loader")
    ap.add_argument("--per-channel", type=int, default=0, choices=[0, 1],
                    help="bert: per-channel weights (DynamicQuantizeLinear -> MatMulInteger -> Cast -> Mul -> Add)")
    ap.add_argument("--memory-planning", type=int, default=1, choices=[0, 1],
                    help="graph configs: time a context whose intermediates share device memory")
    ap.add_argument("--split", type=int, default=2,
                    help="resnet50 / mobilenetv2: the batch as this many slices run concurrently, one "
                         "context and stream each (1: one context for the whole batch)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    runners = {"resnet50": lambda a, d: run_model(a, d, "resnet50"),
               "mobilenetv2": lambda a, d: run_model(a, d, "mobilenetv2"),
               "bert": run_bert, "qoperator": run_qoperator, "bn": run_bn, "convinteger": run_convinteger,
               "qconv": run_qconv, "qmatmul": run_qmatmul, "hbm_copy": run_hbm_copy}
    if args.config == "all":
        res = run_all(args, dev, runners)
    else:
        res = runners[args.config](args, dev)
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": res["dtype"], "data": "synthetic (seeded, BASELINE.json config)",
            "config": res["config"], "roofline": res["roofline"],
            "cpu_baseline": res["cpu_baseline"]}
    if res.get("parity"):
        line["parity"] = res["parity"]
    if res.get("configs"):
        line["configs"] = res["configs"]
    print(json.dumps(line))


if __name__ == "__main__":
    main()
