#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul path (BASELINE.json's metric).

Headline (`value`): the Q4_K decode matvec batch sweep of BASELINE.json
x f32 [B, 2048] ~N(0,1) for B in {1,2,4,8,16}, W [6144, 2048]
~N(0,0.02) quantized to Q4_K.  One "step" is one pass of the sweep (five
qmatmul calls, each on the next of R distinct weight copies, R * 7.08 MB >=
512 MB so the 256 MB Infinity Cache cannot hold them).  `value` is the
algorithmic bytes of the timed steps (weights + x f32 + y f32) divided by the
timed region, in GB/s.  The launches of the
timed steps are replayed from one HIP graph (decode launches are a few
microseconds each; the graph keeps host launch overhead out), bracketed by
HIP events on the stream they run on.

`roofline` is the single-row decode matvec's (C2 at B=1), algorithmic bytes
per launch over its average launch time, with `roofline.also` giving the same
for the B=8 and B=16 calls (activation quantizer + MFMA decode kernel), which
take half of a sweep step; `traffic` is the measured HBM bytes of a call
(profiles/traffic_c2_b*.json).

`details` adds the other BASELINE configs (C1 Q8_0 decode, C3 Q4_K prefill
TFLOP/s, C4 decoder-layer decode, C5 routed experts) measured the same way,
plus the prefill of the Q8_0 and Q6_K weights on their own GEMMs, Q4_K decode
on a 132 MB weight (not launch-bound) and the C5 experts at prefill routing
(512 tokens), and `cpu_baseline` times the C++ restatement of lloom-tensor's CPU QMatMul
(oracle/kq_cpubase.c) on the same weights on a bounded sample.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, 8 TB/s
I8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, 5.0 POP/s
ROTATE_BYTES = 512 << 20   # distinct weight bytes cycled through per config


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-details", action="store_true", help="only the headline config")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="launch only the roofline kernel (C2 at B=1, eagerly, on cold weight copies) and a "
                         "64 MiB device copy, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs")
    ap.add_argument("--pmc-probe-b", type=int, default=1, choices=[1, 2, 4, 8, 16],
                    help="activation rows of the --pmc-probe calls (C2; B >= 5 is two kernels a call)")
    ap.add_argument("--pmc-probe-type", default="q4k", choices=["q4k", "q8_0", "q6k"],
                    help="weight type of --pmc-probe-prefill (q4k: C3's [8192, 2048]; q8_0 [8192, 2048]; "
                         "q6k [2048, 8192])")
    ap.add_argument("--pmc-probe-moe", action="store_true",
                    help="launch only the C5 gate call (routed Q4_K experts, 32 tokens top-8), six times on two "
                         "alternating copies of the experts, for rocprofv3 --pmc runs on the routed kernel")
    ap.add_argument("--pmc-probe-large", action="store_true",
                    help="launch only the Q4_K [28672, 8192] decode (132 MB; --pmc-probe-b rows) on three cold "
                         "weight copies, after a 64 MiB device copy, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs")
    ap.add_argument("--pmc-probe-prefill", action="store_true",
                    help="launch only the C3 prefill GEMM at m=2048 (5 calls), for rocprofv3 --pmc runs on the "
                         "MFMA kernel")
    return ap.parse_args()


class Rotation:
    """R copies of one packed weight in one device buffer (distinct memory)."""

    def __init__(self, qt, copies):
        import torch

        from lloom_amd import QTensor

        size = qt.storage.numel()
        stride = (size + 255) // 256 * 256
        self.buf = torch.empty(stride * copies, dtype=torch.uint8, device=qt.storage.device)
        self.tensors = []
        for i in range(copies):
            view = self.buf[i * stride:i * stride + size]
            view.copy_(qt.storage)
            self.tensors.append(QTensor(view, qt.shape, qt.dtype))

    def __len__(self):
        return len(self.tensors)


def moe_ids(L, np, T, E, topk):
    """C5's routing: top-k of a softmax over seeded uniform logits (synth_uniform(4))."""
    logits = L.synth_uniform(4, T * E).reshape(T, E)
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    return np.argsort(-p, axis=1, kind="stable")[:, :topk].astype(np.int32)


def csrc_digest(names=None):
    """sha256 of kernel sources in lloom_amd/csrc (the named files, or every
    source file; sorted by name).  A committed traffic profile records the
    files its measured kernels are built from and their digest, so a profile
    taken on other kernels is reported as stale, not quoted."""
    import hashlib

    h = hashlib.sha256()
    d = os.path.join(ROOT, "lloom_amd", "csrc")
    for name in sorted(names or os.listdir(d)):
        if name.endswith((".hip", ".hpp", ".cpp", ".h")):
            h.update(name.encode())
            with open(os.path.join(d, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]


def copies_for(packed_bytes):
    return max(2, math.ceil(ROTATE_BYTES / packed_bytes))


def time_graph(fn_list, reps, warmup):
    """Capture fn_list (a list of zero-arg launch callables) into one graph,
    replay it `warmup` times, then time `reps` replays with events.
    Returns seconds per replay."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fn_list:  # eager warm-up (allocations, code objects)
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fn_list:
            f()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / reps


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: every GPU box here has one "
                                   "MI355X; the path would shard by weight rows (or experts), one GPU a shard"}))
        sys.exit(2)
    import numpy as np
    import torch

    import lloom_amd as L

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    lib = L.lib()  # raises if the HIP library is not built

    def cu(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    if args.pmc_probe_moe:
        E, ff, hid, T, topk = 128, 768, 2048, 32, 8
        gate = L.QTensor.quantize(cu(L.synth_normal(40, E * ff * hid, 0.0, 0.02)).view(E, ff, hid), 12)
        copies = [gate, Rotation(gate, 1).tensors[0]]
        ids = moe_ids(L, np, T, E, topk)
        x = cu(L.synth_normal(4000, T * hid)).view(T, 1, hid)
        yg = torch.empty((T, topk, ff), device=dev)
        ids_t = cu(ids)
        for i in range(6):
            copies[i % 2].indexed_moe_forward_into(x, ids_t, yg)
        torch.cuda.synchronize()
        distinct = len(np.unique(ids))
        print(json.dumps({"pmc_probe": "moe_c5_gate", "distinct_experts": distinct,
                          "expert_bytes_per_call": distinct * gate.packed_bytes() // E}))
        return

    # ---------------------------------------------------- headline: C2 ---
    n, k = 6144, 2048
    Bs = [1, 2, 4, 8, 16]
    w = L.synth_normal(1, n * k, 0.0, 0.02)
    qt = L.QTensor.quantize(cu(w).view(n, k), L.GgmlDType.Q4K)
    wbytes = qt.packed_bytes()
    rot = Rotation(qt, copies_for(wbytes))
    xs = {b: cu(L.synth_normal(1000 + b, b * k)).view(b, k) for b in Bs}
    ys = {b: torch.empty((b, n), device=dev) for b in Bs}
    algo = {b: wbytes + b * k * 4 + b * n * 4 for b in Bs}

    counter = [0]

    def launch(b, qtensor):
        return lambda: L.QMatMul(qtensor).forward_into(xs[b], ys[b])

    if args.pmc_probe_prefill:
        dt3 = {"q4k": L.GgmlDType.Q4K, "q8_0": L.GgmlDType.Q8_0, "q6k": L.GgmlDType.Q6K}[args.pmc_probe_type]
        n3, k3, m3 = (2048, 8192, 2048) if args.pmc_probe_type == "q6k" else (8192, 2048, 2048)
        qt3 = L.QTensor.quantize(cu(L.synth_normal(2, n3 * k3, 0.0, 0.02)).view(n3, k3), dt3)
        x3 = cu(L.synth_normal(2000 + m3, m3 * k3)).view(m3, k3)
        y3 = torch.empty((m3, n3), device=dev)
        for _ in range(5):
            L.QMatMul(qt3).forward_into(x3, y3)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": "prefill_%s_m2048" % args.pmc_probe_type, "ops_per_call": 2 * m3 * n3 * k3}))
        return

    if args.pmc_probe_large:
        nl, kl = 28672, 8192
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        qtl = L.QTensor.quantize(cu(L.synth_normal(6, nl * kl, 0.0, 0.02)).view(nl, kl), L.GgmlDType.Q4K)
        rotl = Rotation(qtl, 3)
        pb = args.pmc_probe_b
        xl = cu(L.synth_normal(3000 + pb, pb * kl)).view(pb, kl)
        yl = torch.empty((pb, nl), device=dev)
        for i in range(6):
            L.QMatMul(rotl.tensors[i % 3]).forward_into(xl, yl)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": "large_b%d" % pb, "algorithmic_bytes": qtl.packed_bytes() + pb * (kl + nl) * 4,
                          "copy_bytes": 64 << 20}))
        return

    if args.pmc_probe:
        # the calibration copy (64 MiB read, 64 MiB written), then the kernel
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        pb = args.pmc_probe_b
        for i in range(20):
            launch(pb, rot.tensors[i % len(rot)])()
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": "c2_b%d" % pb, "algorithmic_bytes": algo[pb], "copy_bytes": 64 << 20}))
        return

    sweep = []
    for step in range(args.steps):
        for b in Bs:
            sweep.append(launch(b, rot.tensors[counter[0] % len(rot)]))
            counter[0] += 1
    torch.cuda.synchronize()
    t_step = time_graph(sweep, 1, args.warmup) / args.steps
    step_bytes = sum(algo.values())
    value = step_bytes / t_step / 1e9

    # per-B kernel figures (same method, one B per graph)
    per_b = {}
    for b in Bs:
        fns = [launch(b, rot.tensors[i % len(rot)]) for i in range(len(rot))]
        t = time_graph(fns, 3, 1) / len(fns)
        per_b[str(b)] = {"us": round(t * 1e6, 3), "GB/s": round(algo[b] / t / 1e9, 1),
                         "hbm_frac": round(algo[b] / t / 1e9 / HBM_PEAK_GBS, 4)}

    # the same launches on one copy: weights resident in the 256 MB MALL
    warm = {}
    for b in Bs:
        fns = [launch(b, qt) for _ in range(len(rot))]
        t = time_graph(fns, 3, 1) / len(fns)
        warm[str(b)] = {"us": round(t * 1e6, 3), "GB/s": round(algo[b] / t / 1e9, 1)}
    warm["note"] = "one weight copy replayed: MALL-resident, not an HBM figure"
    # the floor under every per-launch figure: a one-element fill kernel in
    # the same graph timing (the dispatch and completion of one kernel)
    one = torch.empty(1, device=dev)
    t_floor = time_graph([(lambda: one.fill_(1.0)) for _ in range(len(rot))], 3, 1) / len(rot)
    details = {"c2_q4k_decode_per_batch": per_b, "c2_q4k_decode_warm": warm, "rotation_copies": len(rot),
               "rotation_bytes": len(rot) * wbytes,
               "graph_launch_floor_us": {"us": round(t_floor * 1e6, 3),
                                         "note": "a 1-element fill kernel per launch, same graph timing: "
                                                 "the fixed cost in every per-launch figure"}}
    # Roofline of the path's kernels: the single-row decode matvec (C2 at
    # B=1, one kernel a call) and, in `also`, the calls at B=8 and B=16 (the
    # Q8_K activation quantizer, then the MFMA decode kernel), which take half
    # of the sweep's time: algorithmic bytes per call over the call's average
    # time, from the per-B graphs above (events on the replay stream).
    # traffic: measured HBM bytes per call, from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE calibration when present.
    def traffic_of(b):
        """(HBM bytes per launch, or None; where the figure comes from, or why
        it is not quoted: a profile of other kernel sources than these)."""
        tpath = os.path.join(ROOT, "profiles", "traffic_c2_b%d.json" % b)
        if not os.path.exists(tpath):
            return None, "no profile"
        with open(tpath) as f:
            prof = json.load(f)
        digest = csrc_digest(prof.get("digest_files"))
        if prof.get("csrc_digest") != digest:
            return None, "stale: %s measured kernel sources %s (commit %s), these are %s" % (
                os.path.basename(tpath), prof.get("csrc_digest"), prof.get("commit"), digest)
        return prof.get("hbm_bytes_per_launch"), "profiles/%s (commit %s)" % (os.path.basename(tpath),
                                                                            prof.get("commit"))

    def roof(b, kernel):
        t = per_b[str(b)]["us"] * 1e-6
        ach = algo[b] / t / 1e9
        traffic, tnote = traffic_of(b)
        return {"bound": "hbm", "kernel": kernel, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "algorithmic_bytes": algo[b],
                "us_per_launch": per_b[str(b)]["us"], "traffic": traffic, "traffic_source": tnote}

    roofline = roof(1, "k_matvec<Q4_K, 1 row> (C2, B=1)")
    roofline["also"] = [roof(b, "k_quantize_split_q8k + k_mv_dma_ma<8 superblocks, 2 weight tiles, 1 activation "
                                "tile> (C2, B=%d)" % b)
                        for b in (8, 16)]
    del rot
    torch.cuda.empty_cache()

    if not args.no_details:
        details.update(run_details(L, cu, np, torch, dev, args))

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(L, qt, xs, n, k, Bs, algo, args.cpu_seconds)

    line = {
        "metric": "Q4_K/Q8_0 QMatMul decode GB/s (% HBM peak) + prefill TFLOP/s (% i8 MFMA)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4k-weights/q8k-activations (int8 dot4, f32 scales)",
        "data": "synthetic (SplitMix64/xoshiro256** Box-Muller, seeded), random-init weights",
        "config": {"workload": "C2 Q4_K decode matvec sweep, W [6144,2048] Q4_K, x f32 [B,2048], "
                               "B in {1,2,4,8,16}; one step = the 5 calls",
                   "n": n, "k": k, "batches": Bs},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "details": details,
    }
    print(json.dumps(line), flush=True)


def run_details(L, cu, np, torch, dev, args):
    out = {}
    # C1 Q8_0 decode
    n, k = 8192, 2048
    qt = L.QTensor.quantize(cu(L.synth_normal(0, n * k, 0.0, 0.02)).view(n, k), L.GgmlDType.Q8_0)
    rot = Rotation(qt, copies_for(qt.packed_bytes()))
    x = cu(L.synth_normal(1000, k)).view(1, k)
    y = torch.empty((1, n), device=dev)
    t = time_graph([(lambda q=q: L.QMatMul(q).forward_into(x, y)) for q in rot.tensors], 3, 1) / len(rot)
    b = qt.packed_bytes() + k * 4 + n * 4
    out["c1_q8_0_decode"] = {"us": round(t * 1e6, 3), "GB/s": round(b / t / 1e9, 1),
                             "hbm_frac": round(b / t / 1e9 / 8000.0, 4)}
    del rot
    # C3 Q4_K prefill
    n, k = 8192, 2048
    qt = L.QTensor.quantize(cu(L.synth_normal(2, n * k, 0.0, 0.02)).view(n, k), L.GgmlDType.Q4K)
    from lloom_amd.quantized import MMA_AUTO, MMA_F16, MMA_INT8, set_prefill_mma

    # rotating weight copies (>= 512 MB together, past the 256 MB MALL), one
    # call a copy, all of them in one graph: the per-call figure carries
    # neither a cache-resident weight nor a graph launch
    rot3 = Rotation(qt, copies_for(qt.packed_bytes()))
    for mode_name, mode in (("f16", MMA_F16), ("int8", MMA_INT8)):
        set_prefill_mma(mode)
        c3 = {}
        for m in (64, 512, 2048):
            x = cu(L.synth_normal(2000 + m, m * k)).view(m, k)
            y = torch.empty((m, n), device=dev)
            calls = rot3.tensors if m < 2048 else rot3.tensors[:16]
            fns = [lambda t=t: L.QMatMul(t).forward_into(x, y) for t in calls]
            t = time_graph(fns, 3 if m < 2048 else 2, 1) / len(fns)
            ops = 2.0 * m * n * k
            c3[str(m)] = {"us": round(t * 1e6, 2), "TOPS": round(ops / t / 1e12, 2),
                          "i8_peak_frac": round(ops / t / 1e12 / I8_PEAK_TOPS, 4)}
        out["c3_q4k_prefill_" + mode_name] = c3
    set_prefill_mma(MMA_AUTO)
    del rot3
    torch.cuda.empty_cache()
    # prefill of the other weight types on their GEMMs (not a BASELINE
    # config; the C1 Q8_0 weight and the C4 Q6_K down projection, same method)
    for name, dt, n, k in (("q8_0", L.GgmlDType.Q8_0, 8192, 2048), ("q6k", L.GgmlDType.Q6K, 2048, 8192)):
        qt = L.QTensor.quantize(cu(L.synth_normal(5, n * k, 0.0, 0.02)).view(n, k), dt)
        rot = Rotation(qt, copies_for(qt.packed_bytes()))
        pf = {}
        for m in (64, 512, 2048):
            x = cu(L.synth_normal(2000 + m, m * k)).view(m, k)
            y = torch.empty((m, n), device=dev)
            calls = rot.tensors if m < 2048 else rot.tensors[:16]
            fns = [lambda t=t: L.QMatMul(t).forward_into(x, y) for t in calls]
            t = time_graph(fns, 3 if m < 2048 else 2, 1) / len(fns)
            ops = 2.0 * m * n * k
            pf[str(m)] = {"us": round(t * 1e6, 2), "TOPS": round(ops / t / 1e12, 2),
                          "i8_peak_frac": round(ops / t / 1e12 / I8_PEAK_TOPS, 4)}
        out["prefill_" + name + "_%dx%d" % (n, k)] = pf
        del rot
        torch.cuda.empty_cache()
    # decode on a large weight (not a BASELINE config): Q4_K [28672, 8192],
    # 132 MB, the FFN projection of a 70B-class model, where a call is not
    # launch-bound; 4-16 rows (and 2-3 at this size) take the streaming
    # MFMA kernel, one row the dot4 kernel
    n, k = 28672, 8192
    qt = L.QTensor.quantize(cu(L.synth_normal(6, n * k, 0.0, 0.02)).view(n, k), L.GgmlDType.Q4K)
    rot = Rotation(qt, copies_for(qt.packed_bytes()))
    big = {}
    for bsz in (1, 2, 4, 8, 16):
        x = cu(L.synth_normal(3000 + bsz, bsz * k)).view(bsz, k)
        y = torch.empty((bsz, n), device=dev)
        fns = [lambda t=t: L.QMatMul(t).forward_into(x, y) for t in rot.tensors] * 2
        t = time_graph(fns, 3, 1) / len(fns)
        b = qt.packed_bytes() + bsz * (k + n) * 4
        big[str(bsz)] = {"us": round(t * 1e6, 2), "GB/s": round(b / t / 1e9, 1),
                         "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4)}
    for bsz in (1, 16):
        # measured HBM bytes of the call (profiles/traffic_large_b*.json),
        # quoted only for the kernel sources it measured
        tpath = os.path.join(ROOT, "profiles", "traffic_large_b%d.json" % bsz)
        if os.path.exists(tpath):
            with open(tpath) as f:
                prof = json.load(f)
            if prof.get("csrc_digest") == csrc_digest(prof.get("digest_files")):
                big[str(bsz)]["traffic"] = prof.get("hbm_bytes_per_launch")
            else:
                big[str(bsz)]["traffic_source"] = "stale: %s measured other kernel sources" % os.path.basename(tpath)
    big["note"] = "Q4_K [28672, 8192] (132 MB), rotating copies; not a BASELINE config"
    out["decode_q4k_28672x8192"] = big
    del rot
    torch.cuda.empty_cache()
    # C4 decoder layer decode (q,k,v,o,gate,up in Q4_K; down in Q6_K)
    shapes = [("q", 2048, 2048, 12), ("k", 512, 2048, 12), ("v", 512, 2048, 12), ("o", 2048, 2048, 12),
              ("gate", 8192, 2048, 12), ("up", 8192, 2048, 12), ("down", 2048, 8192, 14)]
    layers = []
    total = 0
    for i, (name, nn, kk, dt) in enumerate(shapes):
        q = L.QTensor.quantize(cu(L.synth_normal(30 + i, nn * kk, 0.0, 0.02)).view(nn, kk), dt)
        layers.append((q, nn, kk))
        total += q.packed_bytes()
    ncopy = copies_for(total)
    copies = [[Rotation(q, 1).tensors[0] for (q, _, _) in layers] for _ in range(ncopy)]
    c4 = {}
    for bsz in (1, 4, 16):
        xin = {kk: cu(L.synth_normal(300 + kk, bsz * kk)).view(bsz, kk) for kk in (2048, 8192)}
        yout = {nn: torch.empty((bsz, nn), device=dev) for nn in (512, 2048, 8192)}
        fns = []
        for c in copies:
            for (q, nn, kk), qc in zip(layers, c):
                fns.append(lambda qc=qc, nn=nn, kk=kk: L.QMatMul(qc).forward_into(xin[kk], yout[nn]))
        t = time_graph(fns, 3, 1) / ncopy
        byts = total + sum(bsz * (kk + nn) * 4 for (_, nn, kk) in layers)
        c4[str(bsz)] = {"us_per_layer": round(t * 1e6, 2), "GB/s": round(byts / t / 1e9, 1),
                        "hbm_frac": round(byts / t / 1e9 / 8000.0, 4)}
    out["c4_layer_decode"] = c4
    del copies, layers
    torch.cuda.empty_cache()
    # C5 routed experts: 128 experts, gate/up [768, 2048], down [2048, 768], Q4_K
    E, ff, hid, T, topk = 128, 768, 2048, 32, 8
    gate = L.QTensor.quantize(cu(L.synth_normal(40, E * ff * hid, 0.0, 0.02)).view(E, ff, hid), 12)
    up = L.QTensor.quantize(cu(L.synth_normal(41, E * ff * hid, 0.0, 0.02)).view(E, ff, hid), 12)
    down = L.QTensor.quantize(cu(L.synth_normal(42, E * hid * ff, 0.0, 0.02)).view(E, hid, ff), 12)
    # two copies of the layer's experts (2 x 340 MB), alternated call by
    # call: no expert a call reads is left in the 256 MB MALL by the call
    # before it
    layer_copies = [(gate, up, down), tuple(Rotation(q, 1).tensors[0] for q in (gate, up, down))]
    ids = moe_ids(L, np, T, E, topk)
    ids_t = cu(ids)
    x = cu(L.synth_normal(4000, T * hid)).view(T, 1, hid)
    h = cu(L.synth_normal(4001, T * topk * ff)).view(T, topk, ff)
    yg = torch.empty((T, topk, ff), device=dev)
    yu = torch.empty((T, topk, ff), device=dev)
    yd = torch.empty((T, topk, hid), device=dev)

    def moe_on(g_, u_, d_):
        def moe():
            g_.indexed_moe_forward_into(x, ids_t, yg)
            u_.indexed_moe_forward_into(x, ids_t, yu)
            d_.indexed_moe_forward_into(h, ids_t, yd)
        return moe

    # four passes over the layer a graph replay, on the two copies in turn
    # (the replay's own launch amortized)
    t = time_graph([moe_on(*layer_copies[i % 2]) for i in range(4)], 3, 1) / 4
    distinct = len(np.unique(ids))
    byts = distinct * (gate.packed_bytes() + up.packed_bytes() + down.packed_bytes()) // E
    byts += (T * hid + T * topk * ff) * 4 + (2 * T * topk * ff + T * topk * hid) * 4
    out["c5_moe_experts"] = {"us": round(t * 1e6, 2), "distinct_experts": distinct,
                             "unique_expert_bytes": int(byts), "GB/s": round(byts / t / 1e9, 1),
                             "hbm_frac": round(byts / t / 1e9 / 8000.0, 4),
                             "note": "gate+up+down, 3 routed calls; four passes a graph replay on two "
                                     "alternating copies of the experts (2 x 340 MB)"}

    # the same layer with gate and up as one SwiGLU launch (silu(g) * u
    # stored once) and the down projection over it
    def glu_on(g_, u_, d_):
        def moe_glu():
            g_.indexed_moe_forward_glu_into(u_, x, ids_t, yg)
            d_.indexed_moe_forward_into(yg, ids_t, yd)
        return moe_glu

    t = time_graph([glu_on(*layer_copies[i % 2]) for i in range(4)], 3, 1) / 4
    byts_glu = byts - T * topk * ff * 4  # one [T, topk, ff] store fewer
    out["c5_moe_glu_layer"] = {"us": round(t * 1e6, 2), "GB/s": round(byts_glu / t / 1e9, 1),
                               "hbm_frac": round(byts_glu / t / 1e9 / 8000.0, 4),
                               "note": "silu(gate) * up in one routed launch, then down: 2 routed calls"}
    # the same experts at prefill routing (not a BASELINE config): 512
    # tokens, top-8 from seeded uniform logits; SwiGLU launch + down
    Tp = 512
    lg = L.synth_uniform(5, Tp * E).reshape(Tp, E)
    idp = cu(np.argsort(-lg, axis=1, kind="stable")[:, :topk].astype(np.int32))
    xp = cu(L.synth_normal(4002, Tp * hid)).view(Tp, 1, hid)
    hp = cu(L.synth_normal(4003, Tp * topk * ff)).view(Tp, topk, ff)
    ygp = torch.empty((Tp, topk, ff), device=dev)
    ydp = torch.empty((Tp, topk, hid), device=dev)

    def moe_prefill():
        gate.indexed_moe_forward_glu_into(up, xp, idp, ygp)
        down.indexed_moe_forward_into(hp, idp, ydp)

    t = time_graph([moe_prefill], 5, 1)
    flops = 2.0 * Tp * topk * (2 * ff * hid + hid * ff)
    out["c5_moe_prefill_512"] = {"us": round(t * 1e6, 2), "TFLOP/s": round(flops / t / 1e12, 1),
                                 "note": "512 tokens top-8, SwiGLU launch + down on the C5 experts "
                                         "(dense routing: the fp16-MFMA routed-expert kernel)"}
    return out


def cpu_baseline(L, qt, xs, n, k, Bs, algo, budget_s):
    """The C++ restatement of lloom-tensor's CPU QMatMul (AVX2 vec_dots and the
    barrier-pool driver, oracle/kq_cpubase.c) on the same Q4_K bytes."""
    import numpy as np

    path = os.path.join(ROOT, "oracle", "libkq_cpubase.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.cpb_matmul.argtypes = [ctypes.c_int, sz, sz, sz, vp, vp, vp]
    lib.cpb_pool_init.argtypes = [ctypes.c_int]
    phys = lib.cpb_physical_cores()
    threads = lib.cpb_pool_init(max(1, min(phys, 16)))
    w = np.ascontiguousarray(qt.data())
    xh = {b: np.ascontiguousarray(xs[b].cpu().numpy()) for b in Bs}
    yh = {b: np.empty((b, n), np.float32) for b in Bs}
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    for b in Bs:  # warm-up
        lib.cpb_matmul(12, b, k, n, p(xh[b]), p(w), p(yh[b]))
    iters, t0 = 0, time.perf_counter()
    while True:
        for b in Bs:
            lib.cpb_matmul(12, b, k, n, p(xh[b]), p(w), p(yh[b]))
        iters += 1
        el = time.perf_counter() - t0
        if el >= budget_s or iters >= 2000:
            break
    gbs = iters * sum(algo.values()) / el / 1e9
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": int(threads), "kind": "port",
            "sample": f"C2 sweep B in {{1,2,4,8,16}} x {iters} iterations ({el:.1f} s), same Q4_K bytes, "
                      f"restatement of lloom-tensor CPU QMatMul (AVX2, barrier pool); "
                      f"physical cores {phys}, nproc {os.cpu_count()}, {cpu_model}; one 7 MB weight "
                      f"replayed, so it stays resident in the host caches (the GPU figure streams at least 512 MB "
                      f"of rotating copies from HBM)"}


if __name__ == "__main__":
    main()
